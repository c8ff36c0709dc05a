// Online update of one owned graph (shared by the attention and selection
// kernel files).
#pragma once

#include "ckv_device.h"

namespace ckv {

// Online update of the graph owned by retrieval head rh (no-op for
// non-owners and assignment NONE): exact top-8 merge over the splits'
// candidates, assignment, running-mean centroid, delta append, overflow.
// s_lse0 is the merged lse of the head's first query.  Block size 128..1024
// (the top-8 stage uses the first 512 threads).
//
// Dependent memory rounds: (1) candidates + cursor/count/total and the free
// lists, (2) candidate communities + current key row, (3) per-candidate
// weight/size/delta tail and centroid rows (slot KAPPA holds the community a
// new token would open, or the nearest centroid), (4) every candidate's
// tail-chunk state, in flight during the assignment; then the stores.
// CH: slots each thread loads per round of the top-8 stage (8 or 9; 9 lets
// 512 threads take a 4,096-token budget's 4,235 slots in one round).
// The top-8 stage's first load round (scores and positions of slots
// c * nt + tid, c < CH), issued early by a caller that has a load round of its
// own to overlap it with (the split merge before the update).
template <int CH>
struct Top8First {
  float sv[CH];
  int pv[CH];
};

template <int CH>
__device__ __forceinline__ void top8_first_load(const DecodeArgs& a, const int rh, Top8First<CH>& f) {
  const int tid = threadIdx.x;
  const int nt = min((int)blockDim.x, 512);
  const int scap = a.ws.slot_capacity;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int s = min(c * nt + tid, scap - 1);
    f.sv[c] = gload_f32(a.ws.slot_scores + (int64_t)rh * scap + s);
    f.pv[c] = gload_i32(a.ws.slot_positions + (int64_t)rh * scap + s);
  }
}

template <int CT, int DT, int CH = 8>
__device__ void owner_update(const DecodeArgs& a, const int rh, const float s_lse0,
                             const Top8First<CH>* pre = nullptr) {
  static_assert(CH == 8 || CH == 9, "the top-8 stage sorts 8 or 9 keys per round");
  const int tid = threadIdx.x;
  const int graph = a.st.retrieval_to_graph[rh];
  if (a.cfg.assignment == CKV_ASSIGN_NONE || rh != graph) return;
  __syncthreads();
  CKV_STAMP(rh == 0, 26);

  constexpr int NS = KAPPA + 1;  // candidate slots
  const int C = a.st.community_capacity;
  const int64_t tc_cap = a.st.token_capacity < a.kv.capacity ? a.st.token_capacity : a.kv.capacity;
  const bool delta_q = a.cfg.assignment == CKV_ASSIGN_DELTA_Q;
  const int kvh = a.st.retrieval_to_kv[rh];
  __shared__ uint64_t top[KAPPA];
  __shared__ int s_cur, s_active, s_nearest;
  __shared__ float s_total;
  __shared__ int s_pos[NS], s_comm[NS], s_size[NS], s_dsize[NS], s_tail[NS];
  __shared__ float s_w[NS], s_sc[KAPPA], s_p[KAPPA], s_dw[KAPPA];
  __shared__ float s_key[D];
  __shared__ float s_cent[NS][D];
  __shared__ int s_assigned, s_slot, s_comm_ov;

  // Cursor state and the allocator's free lists, loaded now (in flight with
  // stage 1) and published after it.
  int cur_r = 0, active_r = 0, nearest_r = -1, free_chunk_r = 0, free_pos_r = 0;
  float total_r = 0.0f;
  if (tid == 64) {
    cur_r = a.st.current_position[graph];
    active_r = a.st.community_counts[rh];
    total_r = a.st.total_weight[graph];
    nearest_r = delta_q ? -1 : a.ws.nearest[rh];
  }
  if (tid == 0) {
    free_chunk_r = a.dl.next_free_chunk[graph];
    free_pos_r = a.dl.next_free_position[graph];
  }

  // ---- stage 1: exact top-8 over every attended non-sink slot (score desc,
  // position asc, as one packed 64-bit key each).  Each thread keeps a sorted
  // top-8 of its strided share (loaded CH at a time, one round per chunk;
  // sorted by a 19-comparator network, merged into the running list); each
  // wave then pops its exact top-8 and wave 0 sorts the waves' 64 keys (no
  // thread's or wave's ninth key can be among the head's best eight).
  {
    __shared__ uint64_t wtop[8 * KAPPA];
    const int nt = min((int)blockDim.x, 512);  // threads of this stage
    const int lane = tid & 63, wave = tid >> 6;
    const int scap = a.ws.slot_capacity;
    const float* scs = a.ws.slot_scores + (int64_t)rh * scap;
    const int32_t* sps = a.ws.slot_positions + (int64_t)rh * scap;
    auto cas = [](uint64_t& x, uint64_t& y) {  // x = max, y = min
      const uint64_t hi = x > y ? x : y;
      y = x > y ? y : x;
      x = hi;
    };
    uint64_t loc[KAPPA];
#pragma unroll
    for (int k = 0; k < KAPPA; ++k) loc[k] = 0ull;
    for (int s0 = 0; s0 < scap; s0 += CH * nt) {
      float sv[CH];
      int pv[CH];
      if (s0 == 0 && pre != nullptr) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          sv[c] = pre->sv[c];
          pv[c] = pre->pv[c];
        }
      } else {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
          const int s = min(s0 + c * nt + tid, scap - 1);
          sv[c] = gload_f32(scs + s);
          pv[c] = gload_i32(sps + s);
        }
      }
      uint64_t v[CH];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int s = s0 + c * nt + tid;
        const bool ok = tid < nt && s < scap && s >= a.cfg.num_sink && pv[c] >= 0 && pv[c] < a.kv.capacity;
        v[c] = ok ? pack_candidate(sv[c], pv[c]) : 0ull;
      }
      cas(v[0], v[2]); cas(v[1], v[3]); cas(v[4], v[6]); cas(v[5], v[7]);
      cas(v[0], v[4]); cas(v[1], v[5]); cas(v[2], v[6]); cas(v[3], v[7]);
      cas(v[0], v[1]); cas(v[2], v[3]); cas(v[4], v[5]); cas(v[6], v[7]);
      cas(v[2], v[4]); cas(v[3], v[5]);
      cas(v[1], v[4]); cas(v[3], v[6]);
      cas(v[1], v[2]); cas(v[3], v[4]); cas(v[5], v[6]);
      if constexpr (CH == 9) {  // the ninth key bubbles into the sorted eight
#pragma unroll
        for (int k = 7; k >= 0; --k) cas(v[k], v[k + 1]);
      }
      if (s0 == 0) {
#pragma unroll
        for (int k = 0; k < KAPPA; ++k) loc[k] = v[k];
      } else {
        // top 8 of two sorted lists: pairwise max against the reversed list
        // gives a bitonic sequence of the 8 largest; sort it
#pragma unroll
        for (int k = 0; k < KAPPA; ++k) loc[k] = loc[k] > v[KAPPA - 1 - k] ? loc[k] : v[KAPPA - 1 - k];
        cas(loc[0], loc[4]); cas(loc[1], loc[5]); cas(loc[2], loc[6]); cas(loc[3], loc[7]);
        cas(loc[0], loc[2]); cas(loc[1], loc[3]); cas(loc[4], loc[6]); cas(loc[5], loc[7]);
        cas(loc[0], loc[1]); cas(loc[2], loc[3]); cas(loc[4], loc[5]); cas(loc[6], loc[7]);
      }
    }
    // Exact top-8 of each wave: eight pops of the wave maximum, the lane that
    // held it advancing to its next key (its list is sorted; keys are unique,
    // they hold the position).  The eight waves' lists contain the head's
    // top-8, so one sort of their 64 keys ends the stage.
    for (int r = 0; r < KAPPA; ++r) {
      const uint64_t best = wave_max_u64(loc[0]);
      if (lane == 0 && wave < 8) wtop[wave * KAPPA + r] = best;
      const bool pop = best != 0ull && loc[0] == best;
#pragma unroll
      for (int k = 0; k < KAPPA - 1; ++k) loc[k] = pop ? loc[k + 1] : loc[k];
      loc[KAPPA - 1] = pop ? 0ull : loc[KAPPA - 1];
    }
    __syncthreads();
    if (wave == 0) {
      const int n = (nt >> 6) * KAPPA;  // at most 64 (blocks of at most 512 threads)
      const uint64_t srt = wave_sort_desc_u64(lane < n ? wtop[lane] : 0ull);
      if (lane < KAPPA) top[lane] = srt;
    }
  }
  if (tid == 64) {
    s_cur = cur_r;
    s_active = active_r;
    s_total = total_r;
    s_nearest = nearest_r;
  }
  __syncthreads();
  CKV_STAMP(rh == 0, 27);
  const int cur = s_cur;
  const int active = s_active;
  const bool valid_pos = cur >= 0 && cur < tc_cap;

  // ---- stage 2: candidate communities; the current key row ----------------
  if (tid < NS) {
    int pos = -1, comm = -1;
    if (tid < KAPPA) {
      const uint64_t v = top[tid];
      float sc = NEG_INF;
      if (v != 0ull) {
        sc = unordered_f32((uint32_t)(v >> 32));
        pos = (int)(0xffffffffu - (uint32_t)(v & 0xffffffffu));
      }
      s_sc[tid] = sc;  // (the top-8 outputs are stored at the end: a store here would make
                       // the next loads' completion waits cover it)
      if (delta_q && pos >= 0 && pos < tc_cap) comm = a.st.token_communities[(int64_t)graph * a.st.token_capacity + pos];
    } else {
      comm = (!delta_q && s_nearest >= 0) ? s_nearest : active;  // community a new token would open
    }
    s_pos[tid] = pos;
    s_comm[tid] = comm;
  }
  for (int d = tid; d < D; d += blockDim.x) {
    s_key[d] = valid_pos ? load_elem<DT>(a.kv.key, kvh * a.kv.head_stride + (int64_t)cur * a.kv.token_stride + d) : 0.0f;
  }
  __syncthreads();
  CKV_STAMP(rh == 0, 28);

  // ---- stage 3: per-candidate state and centroid rows ----------------------
  if (tid < NS) {
    const int comm = s_comm[tid];
    const bool ok = comm >= 0 && comm < C;
    s_w[tid] = (ok && delta_q) ? a.st.community_weight[(int64_t)graph * C + comm] : 0.0f;
    s_size[tid] = ok ? a.st.community_sizes[(int64_t)rh * C + comm] : 0;
    s_dsize[tid] = ok ? a.dl.community_sizes[(int64_t)graph * C + comm] : 0;
    s_tail[tid] = ok ? a.dl.community_tail[(int64_t)graph * C + comm] : -1;
  }
  for (int i = tid; i < NS * D; i += blockDim.x) {
    const int k = i / D, d = i % D;
    const int comm = s_comm[k];
    s_cent[k][d] = (comm >= 0 && comm < C) ? load_centroid1<CT>(a.st.centroids, ((int64_t)rh * C + comm) * D + d) : 0.0f;
  }
  __syncthreads();
  CKV_STAMP(rh == 0, 29);

  // Tail-chunk fields of every candidate's community, loaded now (in flight
  // during the assignment) for stage 4, which needs only the assigned one's.
  const int64_t cb = (int64_t)graph * a.dl.chunks_per_graph;
  int t_cs = 0, t_cc = 0, t_st = 0;
  if (tid < NS && a.dl.chunks_per_graph > 0) {
    const int t = s_tail[tid];
    const int tt = min(max(t, 0), a.dl.chunks_per_graph - 1);
    t_cs = gload_i32(a.dl.chunk_size + cb + tt);
    t_cc = gload_i32(a.dl.chunk_capacity + cb + tt);
    t_st = gload_i32(a.dl.chunk_start + cb + tt);
  }

  // ---- assignment (lanes 0..7 of wave 0) ------------------------------------
  if (tid < 64) {
    const int r = tid & 7;
    const int active_c = active < C ? active : C;
    const bool valid = s_pos[r] >= 0 && s_pos[r] < tc_cap;
    const int comm = s_comm[r];
    const bool cand = valid && comm >= 0 && comm < active_c;
    int assigned, slot;
    bool comm_ov;
    if (delta_q) {
      const float half_lam = a.cfg.lam * 0.5f;
      const float p = valid ? ckv_expf(s_sc[r] - s_lse0) : 0.0f;
      const float dw = p * half_lam;
      if (tid < KAPPA) {
        s_p[r] = p;
        s_dw[r] = dw;
      }
      wave_sync();
      // Sequential sums in rank order (reference op order).
      float nd = 0.0f, ssum = 0.0f, sq = 0.0f, cw = 0.0f;
      int first = KAPPA;
#pragma unroll
      for (int j = 0; j < KAPPA; ++j) {
        const float pj = s_p[j], dwj = s_dw[j];
        nd = nd + dwj;
        ssum = ssum + pj;
        sq = sq + pj * pj;
        const int cj = s_comm[j];
        const bool candj = s_pos[j] >= 0 && s_pos[j] < tc_cap && cj >= 0 && cj < active_c;
        if (candj && cj == comm) {
          cw = cw + dwj;
          first = j < first ? j : first;
        }
      }
      const bool leader = cand && first == r;
      const float pair = (ssum * ssum - sq) * (0.5f * (1.0f - a.cfg.lam));
      const float old_total = s_total;
      float two_m = 2.0f * old_total;
      two_m = two_m > 1.0f ? two_m : 1.0f;
      const float oldw = cand ? s_w[r] : 0.0f;
      const float dq = (cand && cw > 0.0f) ? (cw - (nd * oldw) / two_m) : NEG_INF;
      float best = dq;  // max over the 8 lanes of this half-row
      best = fmax_exact(best, ckv_u2f(dpp_u32<0xB1>(ckv_f2u(best))));
      best = fmax_exact(best, ckv_u2f(dpp_u32<0x4E>(ckv_f2u(best))));
      best = fmax_exact(best, ckv_u2f(dpp_u32<0x141>(ckv_f2u(best))));
      int bc = (cand && dq == best) ? comm : 0x7fffffff;
      bc = min(bc, (int)dpp_u32<0xB1>((uint32_t)bc));
      bc = min(bc, (int)dpp_u32<0x4E>((uint32_t)bc));
      bc = min(bc, (int)dpp_u32<0x141>((uint32_t)bc));
      const bool join = best > 0.0f;
      assigned = join ? bc : active;
      comm_ov = assigned >= C;
      // candidate slot that holds the assigned community's prefetched state
      const uint64_t hit = __ballot(tid < KAPPA && comm == assigned);
      slot = join ? (__ffsll((unsigned long long)hit) - 1) : KAPPA;
      if (!comm_ov && tid < KAPPA) {
        if (leader) {
          const float inc = cw + ((join && comm == assigned) ? nd : 0.0f);
          a.st.community_weight[(int64_t)graph * C + comm] = oldw + inc;
        }
        if (tid == 0) {
          if (!join) a.st.community_weight[(int64_t)graph * C + assigned] = nd;
          a.st.community_counts[rh] = active + (join ? 0 : 1);
          a.st.total_weight[graph] = (old_total + nd) + pair;
        }
      }
    } else {
      const int nearest = s_nearest;
      assigned = nearest >= 0 ? nearest : active;
      comm_ov = assigned >= C;
      slot = KAPPA;
      if (tid == 0 && nearest < 0 && !comm_ov) a.st.community_counts[rh] = active + 1;
    }
    if (tid == 0) {
      a.ws.assigned[graph] = comm_ov ? -1 : assigned;
      if (!comm_ov) {
        a.st.community_sizes[(int64_t)rh * C + assigned] = s_size[slot] + 1;
        if (valid_pos) a.st.token_communities[(int64_t)graph * a.st.token_capacity + cur] = assigned;
      }
      s_assigned = assigned;
      s_slot = slot;
      s_comm_ov = comm_ov ? 1 : 0;
    }
  }
  __syncthreads();
  CKV_STAMP(rh == 0, 30);
  const int slot = s_slot;
  const int asg = s_assigned;
  const bool comm_ov = s_comm_ov != 0;
  // Running-mean centroid (FP8 satfinite or f32).
  if (!comm_ov && valid_pos) {
    const int old_size = s_size[slot];
    for (int d = tid; d < D; d += blockDim.x) {
      const float key = s_key[d];
      const float upd = old_size > 0 ? (s_cent[slot][d] * (float)old_size + key) / (float)(old_size + 1) : key;
      store_centroid1<CT>(a.st.centroids, ((int64_t)rh * C + asg) * D + d, upd);
    }
  }
  // ---- stage 4: decode-delta append (the assigned community's tail-chunk
  // fields were prefetched by lane `slot` of wave 0) -------------------------
  int slot_cs = 0, slot_cc = 0, slot_st = 0;
  if (tid < 64) {
    slot_cs = __shfl(t_cs, slot, 64);
    slot_cc = __shfl(t_cc, slot, 64);
    slot_st = __shfl(t_st, slot, 64);
  }
  if (tid == 0) {
    bool chunk_ov = false, pos_ov = false;
    if (!comm_ov) {
      const int64_t tb = (int64_t)graph * C + asg;
      const int delta_size = s_dsize[slot];
      const int old_tail = s_tail[slot];
      const bool tail_ok = old_tail >= 0 && old_tail < a.dl.chunks_per_graph;
      const int old_cs = tail_ok ? slot_cs : 0;
      const int old_cc = tail_ok ? slot_cc : 0;
      const int old_start = tail_ok ? slot_st : 0;
      const int free_chunk = free_chunk_r;
      const int free_pos = free_pos_r;
      const bool allocate = old_tail < 0 || old_cs >= old_cc;
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
        const int start = allocate ? free_pos : old_start;
        const int at = allocate ? 0 : old_cs;
        a.dl.positions[(int64_t)graph * a.dl.position_capacity + start + at] = cur;
        a.dl.chunk_size[cb + chunk] = at + 1;
        a.dl.community_sizes[tb] = delta_size + 1;
      }
    }
    const int overflow = (comm_ov ? 1 : 0) | (chunk_ov ? 2 : 0) | (pos_ov ? 4 : 0) | (valid_pos ? 0 : 8);
    a.ws.overflow[graph] = overflow;
    if (overflow == 0) a.st.current_position[graph] = cur + 1;
  }
  if (tid < KAPPA) {
    a.ws.topk_scores[(int64_t)rh * KAPPA + tid] = s_sc[tid];
    a.ws.topk_positions[(int64_t)rh * KAPPA + tid] = s_pos[tid];
  }
  CKV_STAMP(rh == 0, 31);
}

}  // namespace ckv
