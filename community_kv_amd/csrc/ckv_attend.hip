// Attention over the selected slots, split merge and the fused online update.
#include <type_traits>

#include "ckv_device.h"
#include "ckv_error.h"
#include "ckv_tile.h"
#include "ckv_update.h"

namespace ckv {

namespace {
}  // namespace

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
    a.ws.slot_scores[(int64_t)head * a.ws.slot_capacity + tile * TILE + lane] = s[0];
  }
}

// ---------------------------------------------------------------------------
// Kernel 3: split merge + fused online update
// ---------------------------------------------------------------------------

constexpr int MERGE_MAX_SPLITS = 2048;

// Merges the split partials of query head qh into out/lse with any block size.
// Splits whose max is -inf (no attended slot) are skipped.  Order: the max over
// splits, then sums in split order with the library's deterministic exp/log.
template <int DT>
__device__ inline void merge_head(const DecodeArgs& a, int qh, int tiles, void* out, float* lse_out,
                                  float* lse_keep) {
  __shared__ float scale_s[MERGE_MAX_SPLITS];
  __shared__ float m_s, denom_s;
  const int tid = threadIdx.x;
  const float* pm = a.ws.partial_max + (int64_t)qh * tiles;
  const float* ps = a.ws.partial_sum + (int64_t)qh * tiles;
  __syncthreads();
  if (tid < 64) {
    float M = NEG_INF;
    for (int t = tid; t < tiles; t += 64) M = fmax_exact(M, pm[t]);
    M = wave_max(M);
    if (tid == 0) m_s = M;
  }
  __syncthreads();
  const float M = m_s;
  __shared__ float ls_s[MERGE_MAX_SPLITS];
  for (int t = tid; t < tiles; t += blockDim.x) {
    const float mt = pm[t];
    const float sc = (mt == NEG_INF) ? 0.0f : ckv_expf(mt - M);
    scale_s[t] = sc;
    const float lt = ps[t];
    ls_s[t] = sc != 0.0f ? lt * sc : 0.0f;
  }
  __syncthreads();
  if (tid == 0) {
    float denom = 0.0f;
    for (int t = 0; t < tiles; ++t) denom = denom + ls_s[t];
    denom_s = denom;
  }
  __syncthreads();
  const float* acc_base = a.ws.partial_acc + (int64_t)qh * tiles * D;
  for (int d = tid; d < D; d += blockDim.x) {
    // Loads are unconditional (skipped splits contribute through a select, so
    // stale values of empty splits are never multiplied) and pipelined 8 deep.
    float acc = 0.0f;
    int t = 0;
    for (; t + 8 <= tiles; t += 8) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = acc_base[(int64_t)(t + k) * D + d];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float sc = scale_s[t + k];
        acc = acc + (sc != 0.0f ? v[k] * sc : 0.0f);
      }
    }
    for (; t < tiles; ++t) {
      const float v = acc_base[(int64_t)t * D + d];
      const float sc = scale_s[t];
      acc = acc + (sc != 0.0f ? v * sc : 0.0f);
    }
    const float r = acc / denom_s;
    if constexpr (DT == CKV_BF16) {
      reinterpret_cast<uint16_t*>(out)[(int64_t)qh * D + d] = ckv_f32_to_bf16_bits(r);
    } else {
      reinterpret_cast<float*>(out)[(int64_t)qh * D + d] = r;
    }
  }
  __syncthreads();
  if (tid == 0) {
    const float l = M + ckv_logf(denom_s);
    lse_out[qh] = l;
    if (lse_keep) *lse_keep = l;
  }
}

// Split merge of retrieval head rh's G query heads, one at a time (f32 path).
template <int DT>
__global__ __launch_bounds__(REDUCE_THREADS) void reduce_kernel(DecodeArgs a) {
  const int rh = blockIdx.x;
  const int tiles = a.ws.slot_capacity / TILE;
  for (int g = 0; g < a.cfg.group_size; ++g) {
    merge_head<DT>(a, rh * a.cfg.group_size + g, tiles, a.ws.output, a.ws.lse, nullptr);
  }
}

// Online update of every owned graph, after the attention merge: reads the
// slots' candidate scores and the merged lse of each head's first query.
// 512 threads: the top-8 stage loads a config-2 head's 2,240 slots in one
// round (256 threads needed two; 31.5 -> 29.9 us per layer-step inline).
constexpr int UPDATE_THREADS = 512;
template <int CT, int DT>
__global__ __launch_bounds__(UPDATE_THREADS) void update_kernel(DecodeArgs a) {
  const int rh = blockIdx.x;
  owner_update<CT, DT>(a, rh, a.ws.lse[(int64_t)rh * a.cfg.group_size]);
}

// Batched launches read each item's arguments from a device table
// (workgroup w serves item w / heads, head w % heads).
template <int CT, int DT>
__global__ __launch_bounds__(UPDATE_THREADS) void update_batch_kernel(const DecodeArgs* __restrict__ table, int heads) {
  const DecodeArgs& a = table[blockIdx.x / heads];
  const int rh = blockIdx.x % heads;
  owner_update<CT, DT, 9>(a, rh, a.ws.lse[(int64_t)rh * a.cfg.group_size]);
}

template <int CT, int DT>
__device__ __forceinline__ void sync_shared_body(const DecodeArgs& a, const int rh) {
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

template <int CT, int DT>
__global__ __launch_bounds__(REDUCE_THREADS) void sync_shared_kernel(DecodeArgs a) {
  sync_shared_body<CT, DT>(a, blockIdx.x);
}

template <int CT, int DT>
__global__ __launch_bounds__(REDUCE_THREADS) void sync_shared_batch_kernel(const DecodeArgs* __restrict__ table,
                                                                           int heads) {
  sync_shared_body<CT, DT>(table[blockIdx.x / heads], blockIdx.x % heads);
}

// Merge-only reduce for the dense baseline.
template <int DT>
__global__ __launch_bounds__(REDUCE_THREADS) void dense_reduce_kernel(DecodeArgs a, int tiles) {
  merge_head<DT>(a, blockIdx.x, tiles, a.ws.output, a.ws.lse, nullptr);
}

constexpr int ATT_WAVES = 2;  // waves (one 64-slot tile each) per attention workgroup
constexpr int ATT_TILES = ATT_WAVES;  // 64-slot tiles per attention workgroup

// Split merge of all G query heads of retrieval head rh at once (any block
// size); `scratch` holds 3 * G * splits floats.  When every thread has at most
// two (query, dim) pairs and there are at most 16 splits, the accumulators are
// loaded in the same round as the maxima and sums.
template <int DT>
__device__ inline void merge_group(const DecodeArgs& a, const int rh, const int splits, float* scratch,
                                   float* lse0_out) {
  constexpr int PRE = 16;
  const int tid = threadIdx.x;
  const int nt = blockDim.x;
  const int G = a.cfg.group_size;
  const int n = G * splits;
  float* m_s = scratch;
  float* l_s = scratch + n;
  float* sc_s = scratch + 2 * n;
  __shared__ float gm_s[CKV_MAX_GROUP], gden_s[CKV_MAX_GROUP];
  const int64_t base = (int64_t)rh * G * splits;  // partial_max/sum rows of this head group
  const float* acc_base = a.ws.partial_acc + base * D;
  const bool fast = G * D <= 2 * nt && splits <= PRE;
  float v0[PRE], v1[PRE];
  const int i0 = tid, i1 = tid + nt;
  if (fast) {
    const int p0 = min(i0, G * D - 1), p1 = min(i1, G * D - 1);
    const float* s0 = acc_base + (int64_t)(p0 >> 7) * splits * D + (p0 & (D - 1));
    const float* s1 = acc_base + (int64_t)(p1 >> 7) * splits * D + (p1 & (D - 1));
#pragma unroll
    for (int k = 0; k < PRE; ++k) {
      const int kk = min(k, splits - 1);
      v0[k] = gload_f32(s0 + (int64_t)kk * D);
      v1[k] = gload_f32(s1 + (int64_t)kk * D);
    }
  }
  if (fast && splits <= 16 && 16 * G <= nt) {
    // One row of 16 lanes per query (lane = split): max, scales, denominator
    // and lse by DPP row reductions, published behind a single barrier.
    if (tid < 16 * G) {
      const int g = tid >> 4, t = tid & 15;
      const bool ok = t < splits;
      const float mt = ok ? a.ws.partial_max[base + g * splits + t] : NEG_INF;
      const float lt = ok ? a.ws.partial_sum[base + g * splits + t] : 0.0f;
      float M = mt;
      M = fmax_exact(M, ckv_u2f(dpp_u32<0xB1>(ckv_f2u(M))));
      M = fmax_exact(M, ckv_u2f(dpp_u32<0x4E>(ckv_f2u(M))));
      M = fmax_exact(M, ckv_u2f(dpp_u32<0x141>(ckv_f2u(M))));
      M = fmax_exact(M, ckv_u2f(dpp_u32<0x140>(ckv_f2u(M))));
      const float sc = mt == NEG_INF ? 0.0f : ckv_expf(mt - M);
      float den = sc != 0.0f ? lt * sc : 0.0f;
      den = den + ckv_u2f(dpp_u32<0xB1>(ckv_f2u(den)));
      den = den + ckv_u2f(dpp_u32<0x4E>(ckv_f2u(den)));
      den = den + ckv_u2f(dpp_u32<0x141>(ckv_f2u(den)));
      den = den + ckv_u2f(dpp_u32<0x140>(ckv_f2u(den)));
      if (ok) sc_s[g * splits + t] = sc;
      if (t == 0) {
        gden_s[g] = den;
        const float lse = M + ckv_logf(den);
        a.ws.lse[(int64_t)rh * G + g] = lse;
        if (g == 0 && lse0_out) *lse0_out = lse;
      }
    }
    __syncthreads();
  } else {
    for (int i = tid; i < n; i += nt) {
      m_s[i] = a.ws.partial_max[base + i];
      l_s[i] = a.ws.partial_sum[base + i];
    }
    __syncthreads();
    if (tid < G) {
      float M = NEG_INF;
      for (int t = 0; t < splits; ++t) M = fmax_exact(M, m_s[tid * splits + t]);
      gm_s[tid] = M;
    }
    __syncthreads();
    for (int i = tid; i < n; i += nt) {
      const float mt = m_s[i];
      sc_s[i] = mt == NEG_INF ? 0.0f : ckv_expf(mt - gm_s[i / splits]);
    }
    __syncthreads();
    if (tid < G) {
      float den = 0.0f;
      for (int t = 0; t < splits; ++t) {
        const float sc = sc_s[tid * splits + t];
        den = den + (sc != 0.0f ? l_s[tid * splits + t] * sc : 0.0f);
      }
      gden_s[tid] = den;
      const float lse = gm_s[tid] + ckv_logf(den);
      a.ws.lse[(int64_t)rh * G + tid] = lse;
      if (tid == 0 && lse0_out) *lse0_out = lse;
    }
    __syncthreads();
  }
  auto store = [&](int g, int d, float r) {
    if constexpr (DT == CKV_BF16) {
      reinterpret_cast<uint16_t*>(a.ws.output)[((int64_t)rh * G + g) * D + d] = ckv_f32_to_bf16_bits(r);
    } else {
      reinterpret_cast<float*>(a.ws.output)[((int64_t)rh * G + g) * D + d] = r;
    }
  };
  if (fast) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = h == 0 ? i0 : i1;
      if (i < G * D) {
        const int g = i >> 7;
        const float* scg = sc_s + g * splits;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < PRE; ++k) {
          if (k < splits) acc = acc + (scg[k] != 0.0f ? (h == 0 ? v0[k] : v1[k]) * scg[k] : 0.0f);
        }
        store(g, i & (D - 1), acc / gden_s[g]);
      }
    }
  } else {
    for (int i = tid; i < G * D; i += nt) {
      const int g = i >> 7;
      const int d = i & (D - 1);
      const float* src = acc_base + (int64_t)g * splits * D + d;
      const float* scg = sc_s + g * splits;
      float acc = 0.0f;
      int t = 0;
      for (; t + 16 <= splits; t += 16) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = src[(int64_t)(t + k) * D];
#pragma unroll
        for (int k = 0; k < 16; ++k) acc = acc + (scg[t + k] != 0.0f ? v[k] * scg[t + k] : 0.0f);
      }
      for (; t < splits; ++t) {
        const float v = src[(int64_t)t * D];
        acc = acc + (scg[t] != 0.0f ? v * scg[t] : 0.0f);
      }
      store(g, d, acc / gden_s[g]);
    }
  }
  __syncthreads();
}

// Split merge for up to PRE splits and G * 128 <= 512 outputs: 512 threads,
// one output element per thread with all of its split accumulators loaded up
// front (clamped, one round), and one wave per query reducing max, scales and
// the denominator with lane = split.
constexpr int MERGE_WIDE_THREADS = 512;

// Merged output of one thread (bf16 bits of element tid, tid < G * 128) and
// of lane 0 of waves < G (that query's lse), stored by merge_store: callers
// that load more afterwards store last, so that those loads' completion
// waits do not cover the stores.
struct MergeOut {
  uint16_t bits;
  float lse;
};

// Returns the merged lse of the head's first query (every thread); with
// DEFER the outputs are left in `mo` for merge_store.
template <int PRE, bool DEFER = false>
__device__ __forceinline__ float merge_wide_body(const DecodeArgs& a, const int rh, const int splits,
                                                 MergeOut* mo = nullptr) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int G = a.cfg.group_size;
  const int64_t base = (int64_t)rh * G * splits;
  CKV_STAMP(rh == 0, 24);
  __shared__ float sc_s[MERGE_WIDE_THREADS / 64][PRE];
  __shared__ float den_s[MERGE_WIDE_THREADS / 64];
  __shared__ float lse0_s;
  const int i = min(tid, G * D - 1);
  const float* src = a.ws.partial_acc + (base + (int64_t)(i >> 7) * splits) * D + (i & (D - 1));
  float v[PRE];
#pragma unroll
  for (int k = 0; k < PRE; ++k) v[k] = gload_f32(src + (int64_t)min(k, splits - 1) * D);
  if (wave < G) {
    const bool ok = lane < splits;
    const int64_t j = base + (int64_t)wave * splits + (ok ? lane : 0);
    const float mt = ok ? gload_f32(a.ws.partial_max + j) : NEG_INF;
    const float lt = ok ? gload_f32(a.ws.partial_sum + j) : 0.0f;
    const float M = wave_max(mt);
    const float sc = mt == NEG_INF ? 0.0f : __expf(mt - M);
    const float den = wave_sum_tree(sc != 0.0f ? lt * sc : 0.0f);
    if (lane < PRE) sc_s[wave][lane] = sc;
    if (lane == 0) {
      den_s[wave] = den;
      const float lse = M + __logf(den);
      if constexpr (DEFER) mo->lse = lse; else a.ws.lse[(int64_t)rh * G + wave] = lse;
      if (wave == 0) lse0_s = lse;
    }
  }
  __syncthreads();
  if (tid < G * D) {
    const int g = tid >> 7;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < PRE; ++k) {
      const float sc = sc_s[g][k];
      if (k < splits) acc = acc + (sc != 0.0f ? v[k] * sc : 0.0f);
    }
    const uint16_t bits = ckv_f32_to_bf16_bits(acc / den_s[g]);
    if constexpr (DEFER) mo->bits = bits;
    else reinterpret_cast<uint16_t*>(a.ws.output)[((int64_t)rh * G + g) * D + (tid & (D - 1))] = bits;
  }
  CKV_STAMP(rh == 0, 25);
  return lse0_s;
}

__device__ __forceinline__ void merge_store(const DecodeArgs& a, const int rh, const MergeOut& mo) {
  const int tid = threadIdx.x;
  const int G = a.cfg.group_size;
  if (tid < G * D) reinterpret_cast<uint16_t*>(a.ws.output)[(int64_t)rh * G * D + tid] = mo.bits;
  const int wave = tid >> 6;
  if ((tid & 63) == 0 && wave < G) a.ws.lse[(int64_t)rh * G + wave] = mo.lse;
}

template <int PRE>
__global__ __launch_bounds__(MERGE_WIDE_THREADS) void merge_wide_kernel(DecodeArgs a, int splits) {
  merge_wide_body<PRE>(a, blockIdx.x, splits);
}

template <int PRE>
__global__ __launch_bounds__(MERGE_WIDE_THREADS) void merge_wide_batch_kernel(const DecodeArgs* __restrict__ table,
                                                                              int heads, int splits) {
  merge_wide_body<PRE>(table[blockIdx.x / heads], blockIdx.x % heads, splits);
}

template <int PRE, int CT, int DT>
__global__ __launch_bounds__(MERGE_WIDE_THREADS) void merge_update_kernel(DecodeArgs a, int splits) {
  Top8First<9> pre;  // the update's first load round, in flight with the merge's
  top8_first_load<9>(a, blockIdx.x, pre);
  MergeOut mo;
  const float lse0 = merge_wide_body<PRE, true>(a, blockIdx.x, splits, &mo);
  owner_update<CT, DT, 9>(a, blockIdx.x, lse0, &pre);
  merge_store(a, blockIdx.x, mo);
}

// Split merge and then, in the same workgroup, the head's online update (it
// needs the merged lse of the first query and the slots' candidate scores):
// one kernel boundary fewer than merge + update launches.
template <int PRE, int CT, int DT>
__global__ __launch_bounds__(MERGE_WIDE_THREADS) void merge_update_batch_kernel(
    const DecodeArgs* __restrict__ table, int heads, int splits) {
  const DecodeArgs& a = table[blockIdx.x / heads];
  const int rh = blockIdx.x % heads;
  Top8First<9> pre;  // the update's first load round, in flight with the merge's
  top8_first_load<9>(a, rh, pre);
  MergeOut mo;
  const float lse0 = merge_wide_body<PRE, true>(a, rh, splits, &mo);
  owner_update<CT, DT, 9>(a, rh, lse0, &pre);  // nine slots per thread: one round at config 4
  merge_store(a, rh, mo);
}

// Split merge of the bf16 path: one workgroup per retrieval head.  A kernel of
// its own: on this GPU an agent-scope release/acquire pair around a
// last-arriving-workgroup counter costs more than the kernel boundary.
constexpr int MERGE_SCRATCH = 3 * 1024;  // floats: 3 * G * splits at most

__global__ __launch_bounds__(256) void merge_kernel(DecodeArgs a, int splits) {
  __shared__ __align__(16) float scratch[MERGE_SCRATCH];
  merge_group<CKV_BF16>(a, blockIdx.x, splits, scratch, nullptr);
}

// Sparse bf16 attention: a workgroup of ATT_WAVES waves covers ATT_TILES
// consecutive 64-slot tiles of one retrieval head; each wave runs mfma_tile on
// one tile, the workgroup combines its waves in LDS into one split partial
// (max, sum, unnormalised P.V per query) plus the first query's score of every
// slot (the candidates of the online update's top-8); a separate launch
// merges the splits.
__device__ __forceinline__ void attend_mfma_body(const DecodeArgs& a, const int rh) {
  // Per-wave V half-tile buffers (8 KB each); reused for the waves' P.V rows
  // and, in the last workgroup, as the split-merge scratch.
  __shared__ __align__(16) unsigned char att_dyn[ATT_WAVES * V_HALF_ROWS * D * sizeof(uint16_t)];
  const int wgi = blockIdx.x;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int tid = threadIdx.x;
  const int L = lane >> 4;
  const int c16 = lane & 15;
  const int splits = gridDim.x;
  const int tiles = a.ws.slot_capacity / TILE;
  const int G = a.cfg.group_size;
  const int kvh = a.st.retrieval_to_kv[rh];
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.kv.key);
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.kv.value);
  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.kv.query);
  uint16_t* v_s = reinterpret_cast<uint16_t*>(att_dyn) + wave * (V_HALF_ROWS * D);
  float* o_s = reinterpret_cast<float*>(v_s);  // reused for this wave's P.V rows after the tile

  __shared__ int pos_s[ATT_WAVES][TILE];
  __shared__ float cand_s[ATT_WAVES][TILE];
  __shared__ float wm_s[ATT_WAVES][CKV_MAX_GROUP];
  __shared__ float wl_s[ATT_WAVES][CKV_MAX_GROUP];
  __shared__ float s_lse0;

  const int tile = wgi * ATT_WAVES + wave;
  CKV_STAMP(rh == 0 && wgi == 0, 0);
  const int slot = tile * TILE + lane;
  const bool in_range = tile < tiles;
  int pos = a.ws.slot_positions[(int64_t)rh * a.ws.slot_capacity + (in_range ? slot : 0)];
  const bool valid = in_range && pos >= 0 && pos < a.kv.capacity;
  if (!valid) pos = -1;
  pos_s[wave][lane] = pos;
  const bool any = __ballot(valid) != 0ull;
  const uint4 zero = {0u, 0u, 0u, 0u};
  QOperand qop;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint4 v = gload16(Q + ((int64_t)rh * G + min(c16, G - 1)) * D + 32 * s + 8 * L);
    qop.s[s] = c16 < G ? v : zero;
  }
  wave_sync();
  CKV_STAMP(rh == 0 && wgi == 0, 9);
  const bool want_topk = a.cfg.assignment != CKV_ASSIGN_NONE;
  if (any) {
    f32x4_t o[8];
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) o[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const TileResult r = mfma_tile<2>(K, V, kvh * a.kv.head_stride, a.kv.token_stride, pos_s[wave], v_s,
                                      want_topk ? cand_s[wave] : nullptr, qop, a.cfg.softmax_scale, NEG_INF, o);
    wave_sync();
    CKV_STAMP(rh == 0 && wgi == 0, 1);
    if (L == 0 && c16 < G) {
      wm_s[wave][c16] = r.m;
      wl_s[wave][c16] = r.l;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = 4 * L + i;
      if (g < G) {
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) o_s[g * D + 16 * nb + c16] = o[nb][i];
      }
    }
    // the first query's score of every slot: candidates of the update's top-8
    if (want_topk && in_range) a.ws.slot_scores[(int64_t)rh * a.ws.slot_capacity + slot] = cand_s[wave][lane];
  } else {
    if (L == 0 && c16 < G) {
      wm_s[wave][c16] = NEG_INF;
      wl_s[wave][c16] = 0.0f;
    }
  }
  __syncthreads();
  CKV_STAMP(rh == 0 && wgi == 0, 10);
  // Combine this workgroup's waves into one split partial.
  for (int i = tid; i < G * D; i += 64 * ATT_WAVES) {
    const int g = i >> 7;
    const int d = i & (D - 1);
    float M = NEG_INF;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) M = fmax_exact(M, wm_s[w][g]);
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) {
      const float mw = wm_s[w][g];
      if (mw != NEG_INF) {
        const float* ow = reinterpret_cast<const float*>(reinterpret_cast<uint16_t*>(att_dyn) + w * (V_HALF_ROWS * D));
        acc = acc + ow[g * D + d] * __expf(mw - M);
      }
    }
    a.ws.partial_acc[(((int64_t)rh * G + g) * splits + wgi) * D + d] = acc;
  }
  if (tid < G) {
    float M = NEG_INF;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) M = fmax_exact(M, wm_s[w][tid]);
    float l = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; ++w) {
      const float mw = wm_s[w][tid];
      if (mw != NEG_INF) l = l + wl_s[w][tid] * __expf(mw - M);
    }
    a.ws.partial_max[((int64_t)rh * G + tid) * splits + wgi] = M;
    a.ws.partial_sum[((int64_t)rh * G + tid) * splits + wgi] = l;
  }
  CKV_STAMP(rh == 0 && wgi == 0, 11);
  CKV_STAMP(rh == 0 && wgi == 0, 2);
}

__global__ __launch_bounds__(64 * ATT_WAVES) void attend_mfma_kernel(DecodeArgs a) {
  attend_mfma_body(a, blockIdx.y);
}

__global__ __launch_bounds__(64 * ATT_WAVES) void attend_mfma_batch_kernel(const DecodeArgs* __restrict__ table,
                                                                           int heads) {
  attend_mfma_body(table[blockIdx.y / heads], blockIdx.y % heads);
}

// Dense bf16 decode baseline: each wave streams `chunk_tiles` consecutive
// 64-token tiles of one KV head with an online softmax across tiles and writes
// one split partial per query of its group.
__global__ __launch_bounds__(64) void dense_mfma_kernel(DecodeArgs a, int seq_len, int group, int chunk_tiles) {
  const int chunk = blockIdx.x;
  const int kvh = blockIdx.y;
  const int lane = threadIdx.x;
  const int L = lane >> 4;
  const int c16 = lane & 15;
  const int chunks = gridDim.x;
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.kv.key);
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.kv.value);
  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.kv.query);
  __shared__ __align__(16) uint16_t v_s[V_HALF_ROWS * D];
  __shared__ int pos_s[TILE];
  const uint4 zero = {0u, 0u, 0u, 0u};
  QOperand qop;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint4 v = gload16(Q + ((int64_t)kvh * group + min(c16, group - 1)) * D + 32 * s + 8 * L);
    qop.s[s] = c16 < group ? v : zero;
  }
  f32x4_t o[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) o[nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m = NEG_INF, l = 0.0f;
  for (int t = 0; t < chunk_tiles; ++t) {
    const int base = (chunk * chunk_tiles + t) * TILE;
    if (base >= seq_len) break;
    __syncthreads();
    pos_s[lane] = base + lane < seq_len ? base + lane : -1;
    __syncthreads();
    const TileResult r = mfma_tile<2>(K, V, kvh * a.kv.head_stride, a.kv.token_stride, pos_s, v_s, nullptr, qop,
                                   a.cfg.softmax_scale, m, o);
    const float corr = (m == NEG_INF) ? 0.0f : __expf(m - r.m);
    l = l * corr + r.l;
    m = r.m;
  }
  if (L == 0 && c16 < group) {
    const int qh = kvh * group + c16;
    a.ws.partial_max[(int64_t)qh * chunks + chunk] = m;
    a.ws.partial_sum[(int64_t)qh * chunks + chunk] = l;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int g = 4 * L + i;
    if (g < group) {
      float* dst = a.ws.partial_acc + ((int64_t)(kvh * group + g) * chunks + chunk) * D + c16;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) dst[16 * nb] = o[nb][i];
    }
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

// Split partials per retrieval head written by the attention kernels.
static int attention_splits(const DecodeArgs& a) {
  const int tiles = a.ws.slot_capacity / TILE;
  return a.kv.dtype == CKV_BF16 ? (tiles + ATT_TILES - 1) / ATT_TILES : tiles;
}

// Split merge of `splits` partials per query (bf16 output).
int launch_merge(const DecodeArgs& a, hipStream_t s, int splits) {
  const dim3 mg(a.st.retrieval_heads);
  if (a.cfg.group_size * D <= MERGE_WIDE_THREADS && splits <= 64) {
    if (splits <= 8) hipLaunchKernelGGL(merge_wide_kernel<8>, mg, dim3(MERGE_WIDE_THREADS), 0, s, a, splits);
    else if (splits <= 16) hipLaunchKernelGGL(merge_wide_kernel<16>, mg, dim3(MERGE_WIDE_THREADS), 0, s, a, splits);
    else if (splits <= 32) hipLaunchKernelGGL(merge_wide_kernel<32>, mg, dim3(MERGE_WIDE_THREADS), 0, s, a, splits);
    else if (splits <= 40) hipLaunchKernelGGL(merge_wide_kernel<40>, mg, dim3(MERGE_WIDE_THREADS), 0, s, a, splits);
    else hipLaunchKernelGGL(merge_wide_kernel<64>, mg, dim3(MERGE_WIDE_THREADS), 0, s, a, splits);
  } else {
    if (3 * a.cfg.group_size * splits > MERGE_SCRATCH) {
      return ckv_internal::set_error(CKV_E_LIMIT, "too many attention splits for the merge scratch");
    }
    hipLaunchKernelGGL(merge_kernel, mg, dim3(256), 0, s, a, splits);
  }
  return launch_check("merge");
}

int launch_batch_merge(const DecodeArgs& h, const DecodeArgs* table, int count, int splits, hipStream_t s) {
  const dim3 mg(count * h.st.retrieval_heads);
  const int heads = h.st.retrieval_heads;
  if (splits <= 8) hipLaunchKernelGGL(merge_wide_batch_kernel<8>, mg, dim3(MERGE_WIDE_THREADS), 0, s, table, heads, splits);
  else if (splits <= 16) hipLaunchKernelGGL(merge_wide_batch_kernel<16>, mg, dim3(MERGE_WIDE_THREADS), 0, s, table, heads, splits);
  else if (splits <= 32) hipLaunchKernelGGL(merge_wide_batch_kernel<32>, mg, dim3(MERGE_WIDE_THREADS), 0, s, table, heads, splits);
  else if (splits <= 40) hipLaunchKernelGGL(merge_wide_batch_kernel<40>, mg, dim3(MERGE_WIDE_THREADS), 0, s, table, heads, splits);
  else hipLaunchKernelGGL(merge_wide_batch_kernel<64>, mg, dim3(MERGE_WIDE_THREADS), 0, s, table, heads, splits);
  return launch_check("merge_batch");
}

int launch_attention(const DecodeArgs& a, hipStream_t s, bool partials_only) {
  const int tiles = a.ws.slot_capacity / TILE;
  if (a.kv.dtype == CKV_BF16) {
    const int splits = attention_splits(a);
    if (3 * a.cfg.group_size * splits > MERGE_SCRATCH) {
      return ckv_internal::set_error(CKV_E_LIMIT, "too many attention splits for the merge scratch");
    }
    const dim3 grid(splits, a.st.retrieval_heads);
    hipLaunchKernelGGL(attend_mfma_kernel, grid, dim3(64 * ATT_WAVES), 0, s, a);
    const int r = launch_check("attend_mfma");
    if (r || partials_only) return r;
    return launch_merge(a, s, splits);
  }
  hipLaunchKernelGGL((attend_generic_kernel<CKV_F32, false>), dim3(tiles, a.st.retrieval_heads), dim3(64), 0, s, a, 0,
                     0);
  int r = launch_check("attend");
  if (r || partials_only) return r;
  hipLaunchKernelGGL(reduce_kernel<CKV_F32>, dim3(a.st.retrieval_heads), dim3(REDUCE_THREADS), 0, s, a);
  return launch_check("reduce");
}

// Merge of `splits` bf16 partials (group * 128 <= 512) and the online update
// in one launch, then the shared-graph sync.
int launch_merge_update(const DecodeArgs& a, hipStream_t s, int splits) {
  if (a.cfg.assignment == CKV_ASSIGN_NONE) return launch_merge(a, s, splits);
  const dim3 g(a.st.retrieval_heads);
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, g, dim3(MERGE_WIDE_THREADS), 0, s, a, splits); };
  if (a.st.centroid_dtype == CKV_E4M3) {
    if (splits <= 8) go(merge_update_kernel<8, CKV_E4M3, CKV_BF16>);
    else if (splits <= 16) go(merge_update_kernel<16, CKV_E4M3, CKV_BF16>);
    else if (splits <= 32) go(merge_update_kernel<32, CKV_E4M3, CKV_BF16>);
    else go(merge_update_kernel<64, CKV_E4M3, CKV_BF16>);
  } else {
    if (splits <= 8) go(merge_update_kernel<8, CKV_F32, CKV_BF16>);
    else if (splits <= 16) go(merge_update_kernel<16, CKV_F32, CKV_BF16>);
    else if (splits <= 32) go(merge_update_kernel<32, CKV_F32, CKV_BF16>);
    else go(merge_update_kernel<64, CKV_F32, CKV_BF16>);
  }
  const int r = launch_check("merge_update");
  return r ? r : launch_sync_shared(a, s);
}

int launch_update(const DecodeArgs& a, hipStream_t s) {
  if (a.cfg.assignment == CKV_ASSIGN_NONE) return CKV_OK;
  const bool e4m3 = a.st.centroid_dtype == CKV_E4M3;
  const bool bf16 = a.kv.dtype == CKV_BF16;
  const dim3 g(a.st.retrieval_heads);
  if (e4m3 && bf16) hipLaunchKernelGGL((update_kernel<CKV_E4M3, CKV_BF16>), g, dim3(UPDATE_THREADS), 0, s, a);
  else if (e4m3) hipLaunchKernelGGL((update_kernel<CKV_E4M3, CKV_F32>), g, dim3(UPDATE_THREADS), 0, s, a);
  else if (bf16) hipLaunchKernelGGL((update_kernel<CKV_F32, CKV_BF16>), g, dim3(UPDATE_THREADS), 0, s, a);
  else hipLaunchKernelGGL((update_kernel<CKV_F32, CKV_F32>), g, dim3(UPDATE_THREADS), 0, s, a);
  const int r = launch_check("update");
  return r ? r : launch_sync_shared(a, s);
}

// Layer-wise aggregation: copy the owner's updated community state to the heads sharing its graph.
int launch_sync_shared(const DecodeArgs& a, hipStream_t s) {
  if (a.cfg.assignment == CKV_ASSIGN_NONE || a.st.retrieval_heads == a.st.graph_count) return CKV_OK;
  const bool e4m3 = a.st.centroid_dtype == CKV_E4M3;
  const bool bf16 = a.kv.dtype == CKV_BF16;
  const dim3 g(a.st.retrieval_heads);
  if (e4m3 && bf16) hipLaunchKernelGGL((sync_shared_kernel<CKV_E4M3, CKV_BF16>), g, dim3(REDUCE_THREADS), 0, s, a);
  else if (e4m3) hipLaunchKernelGGL((sync_shared_kernel<CKV_E4M3, CKV_F32>), g, dim3(REDUCE_THREADS), 0, s, a);
  else if (bf16) hipLaunchKernelGGL((sync_shared_kernel<CKV_F32, CKV_BF16>), g, dim3(REDUCE_THREADS), 0, s, a);
  else hipLaunchKernelGGL((sync_shared_kernel<CKV_F32, CKV_F32>), g, dim3(REDUCE_THREADS), 0, s, a);
  return launch_check("sync_shared");
}

int attention_batch_splits(const DecodeArgs& a) {
  const int splits = attention_splits(a);
  return (a.kv.dtype == CKV_BF16 && a.cfg.group_size * D <= MERGE_WIDE_THREADS && splits <= 64) ? splits : 0;
}

// Batched step (bf16 KV): attention + split merge + online update (+ layer-wise
// sync) of `count` items whose DecodeArgs sit in the device table; `h` is the
// host copy of the first item (all items share dtypes, group size, retrieval
// heads and slot capacity).
int launch_batch_attention(const DecodeArgs& h, const DecodeArgs* table, int count, hipStream_t s,
                           bool partials_only) {
  const int heads = h.st.retrieval_heads;
  const int splits = attention_splits(h);
  hipLaunchKernelGGL(attend_mfma_batch_kernel, dim3(splits, count * heads), dim3(64 * ATT_WAVES), 0, s, table,
                     heads);
  int r = launch_check("attend_mfma_batch");
  if (r || partials_only) return r;
  return launch_batch_merge(h, table, count, splits, s);
}

// Layer-wise aggregation of a batch: copy each owner's updated community
// state to the heads sharing its graph.
int launch_batch_sync_shared(const DecodeArgs& h, const DecodeArgs* table, int count, hipStream_t s) {
  const int heads = h.st.retrieval_heads;
  const dim3 g(count * heads);
  if (h.st.centroid_dtype == CKV_E4M3) hipLaunchKernelGGL((sync_shared_batch_kernel<CKV_E4M3, CKV_BF16>), g, dim3(REDUCE_THREADS), 0, s, table, heads);
  else hipLaunchKernelGGL((sync_shared_batch_kernel<CKV_F32, CKV_BF16>), g, dim3(REDUCE_THREADS), 0, s, table, heads);
  return launch_check("sync_shared_batch");
}

int launch_batch_merge_update(const DecodeArgs& h, const DecodeArgs* table, int count, int splits,
                              bool any_shared, hipStream_t s) {
  const int heads = h.st.retrieval_heads;
  const dim3 g(count * heads);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, g, dim3(MERGE_WIDE_THREADS), 0, s, table, heads, splits);
  };
  if (h.st.centroid_dtype == CKV_E4M3) {
    if (splits <= 8) go(merge_update_batch_kernel<8, CKV_E4M3, CKV_BF16>);
    else if (splits <= 16) go(merge_update_batch_kernel<16, CKV_E4M3, CKV_BF16>);
    else if (splits <= 32) go(merge_update_batch_kernel<32, CKV_E4M3, CKV_BF16>);
    else if (splits <= 40) go(merge_update_batch_kernel<40, CKV_E4M3, CKV_BF16>);
    else go(merge_update_batch_kernel<64, CKV_E4M3, CKV_BF16>);
  } else {
    if (splits <= 8) go(merge_update_batch_kernel<8, CKV_F32, CKV_BF16>);
    else if (splits <= 16) go(merge_update_batch_kernel<16, CKV_F32, CKV_BF16>);
    else if (splits <= 32) go(merge_update_batch_kernel<32, CKV_F32, CKV_BF16>);
    else if (splits <= 40) go(merge_update_batch_kernel<40, CKV_F32, CKV_BF16>);
    else go(merge_update_batch_kernel<64, CKV_F32, CKV_BF16>);
  }
  int r = launch_check("merge_update_batch");
  if (r || !any_shared) return r;
  return launch_batch_sync_shared(h, table, count, s);
}

int launch_batch_update(const DecodeArgs& h, const DecodeArgs* table, int count, bool any_shared, hipStream_t s) {
  const int heads = h.st.retrieval_heads;
  const dim3 g(count * heads);
  if (h.st.centroid_dtype == CKV_E4M3) hipLaunchKernelGGL((update_batch_kernel<CKV_E4M3, CKV_BF16>), g, dim3(UPDATE_THREADS), 0, s, table, heads);
  else hipLaunchKernelGGL((update_batch_kernel<CKV_F32, CKV_BF16>), g, dim3(UPDATE_THREADS), 0, s, table, heads);
  int r = launch_check("update_batch");
  if (r || !any_shared) return r;
  return launch_batch_sync_shared(h, table, count, s);
}

int dense_chunks(int seq_len, int chunk_tiles) { return (seq_len + TILE * chunk_tiles - 1) / (TILE * chunk_tiles); }

int launch_dense(const DecodeArgs& a, int seq_len, int group, hipStream_t s) {
  if (a.kv.dtype == CKV_BF16) {
    const int chunk_tiles = CKV_DENSE_CHUNK_TILES;
    const int chunks = dense_chunks(seq_len, chunk_tiles);
    hipLaunchKernelGGL(dense_mfma_kernel, dim3(chunks, a.kv.kv_heads), dim3(64), 0, s, a, seq_len, group, chunk_tiles);
    int r = launch_check("dense_mfma");
    if (r) return r;
    hipLaunchKernelGGL((dense_reduce_kernel<CKV_BF16>), dim3(a.kv.query_heads), dim3(REDUCE_THREADS), 0, s, a, chunks);
    return launch_check("dense_reduce");
  }
  const int tiles = (seq_len + TILE - 1) / TILE;
  hipLaunchKernelGGL((attend_generic_kernel<CKV_F32, true>), dim3(tiles, a.kv.kv_heads), dim3(64), 0, s, a, seq_len, group);
  int r = launch_check("dense attend");
  if (r) return r;
  hipLaunchKernelGGL((dense_reduce_kernel<CKV_F32>), dim3(a.kv.query_heads), dim3(REDUCE_THREADS), 0, s, a, tiles);
  return launch_check("dense reduce");
}

}  // namespace ckv

#ifdef CKV_PHASE_TIMING
extern "C" int ckv_phase_stamps_attend(unsigned long long* out) {
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(ckv::phase_stamp), sizeof(unsigned long long) * 32);
}
#endif
