// Centroid scoring + exact community selection + slot materialisation, and
// the fused selection + attention launch.
//
// select_body: one 512-thread workgroup per retrieval head.  Every decode
// layer-step is a chain of dependent memory round trips, so the body is laid
// out to need as few of them as possible:
//   R0  head mapping, query group, centroid rows, community sizes, sinks
//   R1  graph-indexed fields of every scored community: CSR start, decode-delta
//       member count and tail chunk (in flight during the scoring)
//   --  scoring as soon as R0 has landed
//   R2  tail-chunk start and fill of every community with decode deltas, and
//       the communities of the window tokens (issued after the scoring, in
//       flight during the selection)
//   --  exact weighted selection and descriptors
//   R3  one gather round for the attended slots (CSR member, delta member)
// Scoring: 8 lanes per centroid row (16 dims each), pinned fp32 summation order
// (each lane sums its 16 products in order, then a butterfly over the 8 lanes),
// fp16 round-to-nearest-even key.  Selection: two 8-bit radix passes over
// order-preserving fp16 keys in LDS, descriptors in the reference order.
//
// Kernels: select_kernel (the selection alone: writes the slot table for the
// attention kernels), select_attend_kernel (FUSED: parts workgroups per head
// each run the selection, resolve only their own two tiles' slots and attend
// them into split partials), their batched variants over a device table of
// items, and select_prescored_batch_kernel (scores computed beforehand by
// score_rows_batch_kernel on every compute unit).  Workgroups past the heads
// run the deferred online update of another layer.
//
// Reference: attention/kernels/centroid_selection.py:32-188 (scoring),
// attention/kernels/_csrc/descriptor_selection.cu:164-487 (selection),
// attention/kernels/segmented_attention.py:98-282 (slot -> position mapping).
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "ckv_device.h"
#include "ckv_error.h"
#include "ckv_tile.h"
#include "ckv_update.h"
#include "ckv_score.h"

#ifndef CKV_R2_LATE
#define CKV_R2_LATE 0
#endif
namespace ckv {

namespace {

int limit_error(const char* message) { return ckv_internal::set_error(CKV_E_LIMIT, message); }

constexpr int ROWS_PER_PASS = SELECT_THREADS / 8;          // centroid rows scored per pass
constexpr int MAT_BATCH = 8;                               // 64-slot blocks per wave gathered together
constexpr int DESC_ARRAYS = 7;                             // per-descriptor LDS arrays
// Dynamic LDS the fused kernel may use: a workgroup's 160 KB less the static
// arrays (up to 24 KB in the fused instances, by the compiler's resource
// report), with 2 KB to spare.
constexpr size_t FUSED_LDS_LIMIT = 134 * 1024;
// 64-slot tiles attended per workgroup of the fused path (parts per head = tiles / this).
constexpr int FUSED_TILES = 2;
// Cooperative fused launch: polling rounds (each a memory round trip plus a
// short sleep, about 1 us) before a part scores the missing communities
// itself; at most 64 parts per head.
constexpr int COOP_POLLS = 64;
constexpr int COOP_PRE = 2;  // passes of the cooperative scoring share loaded with the first round
constexpr int COOP_SCORE_WAVES = 6;  // waves that score and poll; the others walk the graph-indexed chain
constexpr int COOP_MAX_PARTS = 64;
// Separate (non-fused) selections: workgroups per head at most, and the
// compute units one round of them should fill (MI355X: 256).
#ifndef CKV_PRESELECT_MAX_PARTS
#define CKV_PRESELECT_MAX_PARTS 4
#endif
constexpr int PRESELECT_MAX_PARTS = CKV_PRESELECT_MAX_PARTS;
constexpr int64_t CKV_DEVICE_CUS = 256;
constexpr int COOP_WAVES = SELECT_THREADS / 64;
// Exchange row layout after the C tagged scores: the nearest-centroid minima
// (part * COOP_WAVES + wave), then COOP_MAX_PARTS * COOP_WAVES reserved words.
constexpr int COOP_NEAR_OFF = 0;
}  // namespace

__host__ __device__ inline int64_t exchange_stride(int community_capacity) {
  return ckv_exchange_words(community_capacity);
}
// Low 16 bits of a launch's tag, carried by the nearest-centroid minima.
__device__ inline uint64_t near_tag16(uint32_t epoch) { return (uint64_t)((epoch + 1u) & 0xffffu); }

// Arrival of one part of head rh.  The last part to arrive merges the head's
// split partials into output and lse (the arithmetic of merge_wide_body, so
// the results equal the separate merge kernel's), reduces the parts'
// nearest-centroid minima into a.ws.nearest, then resets the arrival counter
// and advances the head's epoch for the next launch.  Nothing here waits on
// another workgroup.
template <int PMAX>
__device__ __forceinline__ void coop_finish(const DecodeArgs& a, const int rh, const int parts, const uint32_t epoch,
                                            const bool nearest_mode, const uint64_t* xrow) {
  __shared__ int s_last;
  __shared__ float sc_s[CKV_MAX_GROUP][PMAX];
  __shared__ float den_s[CKV_MAX_GROUP];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  uint32_t* counter = a.ws.block_counters + rh;
  CKV_STAMP_MAX(rh == 0, 29);
  // Every wave's partial stores (agent-scope, written through) complete
  // before the barrier; the barrier orders them before thread 0's agent-scope
  // release increment (workgroup synchronisation, then agent
  // synchronisation).  Increments continue the counter's release sequence, so
  // the part that reads parts - 1 acquires every other part's stores with an
  // agent-scope acquire fence, before the barrier that lets its threads load
  // the partials.  Release/acquire in the language's terms, valid whichever
  // XCDs the parts run on.  (Measured at config 2: 16.70 against 16.58 us per
  // layer-step with a relaxed increment; an acq_rel increment in every part,
  // whose acquire invalidates the XCD's L2 once per part, 17.09 us; an
  // agent-scope release fence in every thread, one L2 write-back per wave,
  // 25.5 us.)
  wait_vm();
  __syncthreads();
  if (tid == 0) {
    const bool last =
        __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)(parts - 1);
    if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;
  CKV_STAMP(rh == 0, 24);
  const int G = a.cfg.group_size;
  const int C = a.st.community_capacity;
  const int64_t base = (int64_t)rh * G * parts;
  const int i = min(tid, G * D - 1);
  const float* src = a.ws.partial_acc + (base + (int64_t)(i >> 7) * parts) * D + (i & (D - 1));
  // the maxima and sums first: their reduction runs while the accumulators arrive
  const bool ok = wave < G && lane < parts;
  const int64_t j = base + (int64_t)min(wave, G - 1) * parts + (ok ? lane : 0);
  const float mt0 = ld_agent_f32(a.ws.partial_max + j);
  const float lt0 = ld_agent_f32(a.ws.partial_sum + j);
  float v[PMAX];
#pragma unroll
  for (int k = 0; k < PMAX; ++k) v[k] = ld_agent_f32(src + (int64_t)min(k, parts - 1) * D);
  if (wave < G) {
    const float mt = ok ? mt0 : NEG_INF;
    const float lt = ok ? lt0 : 0.0f;
    const float M = wave_max(mt);
    const float sc = mt == NEG_INF ? 0.0f : __expf(mt - M);
    const float den = wave_sum_tree(sc != 0.0f ? lt * sc : 0.0f);
    if (lane < PMAX) sc_s[wave][lane] = sc;
    if (lane == 0) {
      den_s[wave] = den;
      a.ws.lse[(int64_t)rh * G + wave] = M + __logf(den);
    }
  } else if (nearest_mode && wave == COOP_WAVES - 1) {
    // distance bits << 32 | row << 16 | tag; every part's stores have landed
    uint64_t m = ~0ull;
    for (int e = lane; e < parts * COOP_WAVES; e += 64) {
      const uint64_t x = ld_agent_u64(xrow + C + COOP_NEAR_OFF + e);
      m = x < m ? x : m;
    }
    m = wave_min_u64(m);
    if (lane == 0) a.ws.nearest[rh] = (m >> 32) == 0xffffffffull ? -1 : (int)((m >> 16) & 0xffffu);
  }
  __syncthreads();
  if (tid < G * D) {
    const int g = tid >> 7;
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < PMAX; ++k) {
      const float sc = sc_s[g][k];
      if (k < parts) acc = acc + (sc != 0.0f ? v[k] * sc : 0.0f);
    }
    reinterpret_cast<uint16_t*>(a.ws.output)[((int64_t)rh * G + g) * D + (tid & (D - 1))] =
        ckv_f32_to_bf16_bits(acc / den_s[g]);
  }
  if (tid == 0) {
    st_agent_u32(counter, 0u);
    st_agent_u32(a.ws.block_counters + 2 * a.st.retrieval_heads + rh, epoch + 1u);
  }
  CKV_STAMP(rh == 0, 25);
  CKV_STAMP_MAX(true, 30);
}

// OWN: communities owned per thread (thread t owns [t*OWN, (t+1)*OWN), so id
// order is thread order then k order), chosen from the scored community count
// so that the per-community fields stay in registers.  Workgroups beyond
// a.st.retrieval_heads run the pending online update of another layer `u`
// (same dtypes, disjoint state) on otherwise idle CUs.
// LDS bytes of the fused path's slot table (16-byte aligned).
__host__ __device__ inline size_t fused_slot_bytes(int slot_capacity) { return ((size_t)slot_capacity * 4 + 15) & ~(size_t)15; }
// LDS of the fused path's selection (16-byte aligned), after the window
// communities: fp16 keys, seven per-community int arrays (selection start,
// size, CSR start, delta count, tail chunk, its start and fill) and the tile
// marks; the attention buffers follow.
__host__ __device__ inline size_t fused_select_bytes(int community_capacity, int budget_tiles, int parts) {
  const size_t cp = (size_t)((community_capacity + 7) & ~7);
  const size_t td = (size_t)((budget_tiles + parts - 1) / parts);
  return (cp * 2 + cp * 8 * 4 + ((size_t)FUSED_TILES * TILE + td) * 4 + 15) & ~(size_t)15;
}
__device__ inline int* fused_fields(unsigned char* dyn, int community_capacity) {
  return reinterpret_cast<int*>(dyn + (size_t)((community_capacity + 7) & ~7) * 2);
}
__device__ inline int* fused_marks(unsigned char* dyn, int community_capacity) {
  return fused_fields(dyn, community_capacity) + 8 * ((community_capacity + 7) & ~7);
}

// FUSED: `part` of `parts` workgroups of this head each run the whole
// selection (they are latency-bound, so the copies cost no time), resolve the
// slots of their own tiles only, attend them (attend_part) and write that
// part of the slot table; the selection's other outputs are split over the
// parts.
// PRE: the scores were written to a.ws.scores by score_rows_kernel (no
// nearest-centroid search then); the workgroup loads them instead of scoring.
// COOP (with FUSED): each part scores only its share of the live communities
// and publishes it, epoch-tagged, in a.ws.exchange; the parts read the other
// shares from there (bounded polling: a part that does not see them all
// within COOP_POLLS rounds scores every community itself, so no part waits
// on another indefinitely).  The last part to finish merges the head's split
// partials (coop_finish).
template <int CT, int DT, int OWN, bool FUSED = false, bool PRE = false, bool COOP = false, int PMAX = 32>
__device__ __forceinline__ void select_body(const DecodeArgs& a, const int rh, const int part = 0,
                                            const int parts = 1) {
  constexpr int PB = CT == CKV_E4M3 ? 4 : 2;  // scoring passes whose loads are in flight together
  constexpr int WAVES = SELECT_THREADS / 64;
  constexpr int WIN_PER_THREAD = (CKV_MAX_WINDOW + SELECT_THREADS - 1) / SELECT_THREADS;
  const int tid = threadIdx.x;
  const int G = a.cfg.group_size;
  const int C = a.st.community_capacity;
  const int nscore = min(C, a.ws.score_blocks * SCORE_BLOCK);
  const bool nearest_mode = a.cfg.assignment == CKV_ASSIGN_NEAREST;
  const bool materialise = a.csr.member_offsets != nullptr;
  const int ns = a.cfg.num_sink;
  const int W = a.cfg.local_window;
  const int cpg = a.dl.chunks_per_graph;
  CKV_TS_DECL;
  CKV_TS(0);
  CKV_STAMP_MAX(FUSED && rh == 0, 26);

  __shared__ float q_s[CKV_MAX_GROUP * D];
  __shared__ float key_s[D];
  __shared__ __align__(16) int hist[256];
  __shared__ __align__(16) int hist2[256];  // second radix pass (no clearing barrier in between)
  __shared__ __align__(16) int scan_s[4 * WAVES * OWN];
  __shared__ uint64_t near_s[WAVES];
  __shared__ int sink_s[CKV_MAX_SINKS];
  __shared__ int s_max_idx, s_sel_count, s_last_sel_pos, s_last_size, s_sink_max, s_cur;

  extern __shared__ __align__(16) unsigned char dyn_all[];
  // fused: the window tokens' communities first, then the selection arrays (later the attention buffers)
  int* slot_lds = reinterpret_cast<int*>(dyn_all);
  unsigned char* dyn = dyn_all + (FUSED ? fused_slot_bytes(a.ws.slot_capacity) : 0);
  uint16_t* key16 = reinterpret_cast<uint16_t*>(dyn);  // masked fp16 score bits of every scored community
  const int dcap = a.ws.descriptor_capacity;
  // (unfused: the key table holds the scored rows only, so a large capacity
  // with few scored rows keeps the LDS small)
  int* desc_comm = reinterpret_cast<int*>(dyn + (size_t)(((FUSED ? C : nscore) + 7) & ~7) * 2);
  int* desc_end = desc_comm + dcap;  // cumulative selected-token end
  int* desc_lo = desc_end + dcap;    // CSR start of the community
  int* desc_dc = desc_lo + dcap;     // decode-delta member count
  int* desc_tl = desc_dc + dcap;     // tail chunk id
  int* desc_ts = desc_tl + dcap;     // tail chunk start
  int* desc_tn = desc_ts + dcap;     // tail chunk fill
  int* blk_first = desc_tn + dcap;   // descriptor holding the first slot of each 64-slot block of the selection

  // Every prefetch load below is unconditional (indices clamped, results
  // masked afterwards) and no global store is issued before the last gather:
  // loads and stores share one completion counter, so a branch around a load
  // or an early store would make later waits cover them too.

  // ---- R0 -------------------------------------------------------------------
  int count = a.st.community_counts[rh];
  const int graph = a.st.retrieval_to_graph[rh];
  const int kvh = a.st.retrieval_to_kv[rh];
  count = count < 0 ? 0 : (count > nscore ? nscore : count);

  const int sub = tid >> 3;
  const int lane8 = tid & 7;
  const int passes = (nscore + ROWS_PER_PASS - 1) / ROWS_PER_PASS;
  // Two batches of centroid fragments: the next batch's loads are in flight
  // while the current one is scored.
  CentroidFrag<CT> frag[2][PB];
  int rsize[2][PB];
  auto load_batch = [&](int p0, int buf, int last_row) {
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
      const int row = min((p0 + pb) * ROWS_PER_PASS + sub, last_row);
      load_frag<CT>(a.st.centroids, (int64_t)rh * C + row, 16 * lane8, frag[buf][pb]);
      rsize[buf][pb] = gload_i32(a.st.community_sizes + (int64_t)rh * C + row);
    }
  };
  if constexpr (!PRE && !COOP) {
    load_batch(0, 0, nscore - 1);
    load_batch(PB, 1, nscore - 1);  // clamped rows: harmless when there is no second batch
  }
  // COOP: waves 0 .. COOP_SCORE_WAVES - 1 score this part's share of the rows
  // and poll for the other parts' shares; the remaining waves walk the
  // graph-indexed chain (CSR offsets, decode-delta fields, tail chunks, window
  // communities, sinks, current key) into LDS, so that the scoring waves' memory
  // waits never cover those dependent rounds.  The share is interleaved (rows
  // part, part + parts, ...), so its addresses do not wait for the community
  // count, and up to COOP_PRE passes of fragments are loaded with the first
  // round.  Each row's 8-lane group is replicated over `qps` query-pair groups
  // (thread bits 3..), which split the query pairs of the group between them.
  uint64_t* xrow = COOP ? a.ws.exchange + (int64_t)rh * exchange_stride(C) : nullptr;
  uint32_t epoch = 0;
  const bool chain_wave = COOP && (tid >> 6) >= COOP_SCORE_WAVES;
  // Blocks go to the eight XCDs round robin and the parts of head rh are blocks
  // rh + R * part, so with R a multiple of 8 they share one XCD: the scores
  // then stay in its L2 (st_xcd_u64), else they are written through.
  const bool xcd_local = (a.st.retrieval_heads & 7) == 0;
  const int npairs = (G + 1) >> 1;
  const int rpp = (nscore + max(parts, 1) - 1) / max(parts, 1);  // rows per part
  int qps_log = 0;
  if constexpr (COOP) {
    const int pairs_log = npairs <= 1 ? 0 : 1;  // the fused path serves groups of at most four queries
    for (int l = pairs_log; l > 0; --l) {
      if (((COOP_SCORE_WAVES * 64) >> (3 + l)) >= rpp) {
        qps_log = l;
        break;
      }
    }
  }
  const int qp = (tid >> 3) & ((1 << qps_log) - 1);
  const int ri = tid >> (3 + qps_log);  // row of this thread within a pass
  const int rows_pass = (COOP_SCORE_WAVES * 64) >> (3 + qps_log);
  CentroidFrag<CT> cfrag[COOP_PRE];
  int csize[COOP_PRE];
  uint4 qraw[2][2][2];  // [pair][query of the pair][dims 0-7, 8-15 of this lane's slice], bf16
  if constexpr (COOP) {
    epoch = ld_agent_u32(a.ws.block_counters + 2 * a.st.retrieval_heads + rh);
    if (!chain_wave) {
#pragma unroll
      for (int ps = 0; ps < COOP_PRE; ++ps) {
        const int row = min(part + parts * min(ri + ps * rows_pass, rpp - 1), nscore - 1);
        load_frag<CT>(a.st.centroids, (int64_t)rh * C + row, 16 * lane8, cfrag[ps]);
        csize[ps] = gload_i32(a.st.community_sizes + (int64_t)rh * C + row);
      }
      const uint16_t* qbase = reinterpret_cast<const uint16_t*>(a.kv.query) + (int64_t)rh * G * D + 16 * lane8;
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int g = min(2 * qp + (2 << qps_log) * j + u, G - 1);
          qraw[j][u][0] = gload16(qbase + (int64_t)g * D);
          qraw[j][u][1] = gload16(qbase + (int64_t)g * D + 8);
        }
      }
    }
  }
  const uint64_t tag = (uint64_t)(epoch + 1u) << 32;
  // Query group: two elements per thread (G * 128 <= 2048 <= 4 * threads).
  float qv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  // prescored: the scores of this head's rows t, t + threads, ...
  uint16_t pre_key[OWN];
  if constexpr (PRE) {
#pragma unroll
    for (int k = 0; k < OWN; ++k)
      pre_key[k] = reinterpret_cast<const uint16_t*>(a.ws.scores)[(int64_t)rh * C +
                                                                    min(tid + k * SELECT_THREADS, nscore - 1)];
  }
#pragma unroll
  for (int h = 0; h < ((PRE || COOP) ? 0 : 2); ++h) {
    const int qe = min(2 * (tid + h * SELECT_THREADS), G * D - 2);
    if constexpr (DT == CKV_BF16) {
      const uint32_t w = (uint32_t)gload_i32(reinterpret_cast<const int32_t*>(
          reinterpret_cast<const uint16_t*>(a.kv.query) + (int64_t)rh * G * D + qe));
      qv[2 * h] = ckv_u2f(w << 16);
      qv[2 * h + 1] = ckv_u2f(w & 0xffff0000u);
    } else {
      const float* qp = reinterpret_cast<const float*>(a.kv.query) + (int64_t)rh * G * D + qe;
      qv[2 * h] = gload_f32(qp);
      qv[2 * h + 1] = gload_f32(qp + 1);
    }
  }
  const int sink_v = (!COOP && materialise && ns > 0) ? gload_i32(a.cfg.sink_positions + min(tid, ns - 1)) : -1;
  // thread t owns communities t, t + SELECT_THREADS, ...: id order is k, then thread
  auto cid = [&](int k) { return tid + k * SELECT_THREADS; };
  int o_size[OWN];
#pragma unroll
  for (int k = 0; k < OWN; ++k) o_size[k] = gload_i32(a.st.community_sizes + (int64_t)rh * C + min(cid(k), nscore - 1));

  // ---- R1 -------------------------------------------------------------------
  int cur = COOP ? 0 : a.st.current_position[graph];  // COOP: from LDS after the polls
  const int64_t tbl = (int64_t)graph * C;
  const int64_t cb = (int64_t)graph * cpg;
  int o_lo[OWN], o_dc[OWN], o_tl[OWN], o_ts[OWN], o_tn[OWN];
#pragma unroll
  for (int k = 0; k < OWN; ++k) {
    o_lo[k] = 0;
    o_dc[k] = 0;
    o_tl[k] = -1;
    o_ts[k] = 0;
    o_tn[k] = 0;
  }
  if (!COOP && materialise) {
#pragma unroll
    for (int k = 0; k < OWN; ++k) {
      const int c = min(cid(k), C - 1);
      o_lo[k] = gload_i32(a.csr.member_offsets + (int64_t)graph * (C + 1) + c);
      o_dc[k] = gload_i32(a.dl.community_sizes + tbl + c);
      o_tl[k] = gload_i32(a.dl.community_tail + tbl + c);
    }
  }
  float key_v = 0.0f;
  if (!COOP && nearest_mode) {
    const int64_t cp = cur < 0 ? 0 : (cur >= a.kv.capacity ? a.kv.capacity - 1 : cur);
    key_v = load_elem<DT>(a.kv.key, kvh * a.kv.head_stride + cp * a.kv.token_stride + (tid & (D - 1)));
  }

  if constexpr (!COOP) {  // (COOP: the chain waves set these up)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = 2 * (tid + h * SELECT_THREADS);
      if (e < G * D) {
        q_s[e] = qv[2 * h];
        q_s[e + 1] = qv[2 * h + 1];
      }
    }
    if (tid < ns) sink_s[tid] = sink_v;
    if (nearest_mode && tid < D) key_s[tid] = (cur >= 0 && cur < a.kv.capacity) ? key_v : 0.0f;
    hist[tid & 255] = 0;
    hist2[tid & 255] = 0;
    if (tid == 0) {
      s_max_idx = -1;
      s_sel_count = 0;
    }
    if constexpr (FUSED) {  // tile marks (see the fused slot resolution)
      if (tid < FUSED_TILES * TILE) fused_marks(dyn, C)[tid] = -1;
    }
  }
  // R2 issue (tail-chunk start and fill of every owned community with decode
  // deltas, the communities of the window tokens).  The cooperative path
  // issues it right after R0 lands (its scoring share was loaded before, and
  // the polls after it take as long), the others after the scoring.
  int wcomm[WIN_PER_THREAD];
#pragma unroll
  for (int h = 0; h < WIN_PER_THREAD; ++h) wcomm[h] = -1;
  auto issue_r2 = [&]() {
    if (!materialise) return;
    if (cpg > 0) {
#pragma unroll
      for (int k = 0; k < OWN; ++k) {
        const int t = min(max(o_tl[k], 0), cpg - 1);
        o_ts[k] = gload_i32(a.dl.chunk_start + cb + t);
        o_tn[k] = gload_i32(a.dl.chunk_size + cb + t);
      }
    }
    if (W > 0) {
      const int32_t* tcomm = a.st.token_communities + (int64_t)graph * a.st.token_capacity;
#pragma unroll
      for (int h = 0; h < WIN_PER_THREAD; ++h) {
        const int64_t p = (int64_t)cur - W + tid + h * SELECT_THREADS;
        wcomm[h] = gload_i32(tcomm + (p < 0 ? 0 : (p >= a.st.token_capacity ? a.st.token_capacity - 1 : p)));
      }
    }
  };
  if constexpr (!COOP) __syncthreads();  // q_s, key_s, sink_s, hist
  if constexpr (!COOP) CKV_TS(6);
  if (!COOP && tid < 64) {  // largest sink position: window tokens beyond it skip the sink test
    int m = -1;
    for (int i = tid; i < ns; i += 64) m = max(m, sink_s[i]);
    m = max(m, (int)dpp_u32<0xB1>((uint32_t)m));
    m = max(m, (int)dpp_u32<0x4E>((uint32_t)m));
    m = max(m, (int)dpp_u32<0x141>((uint32_t)m));
    m = max(m, (int)dpp_u32<0x140>((uint32_t)m));
    m = max(m, __builtin_amdgcn_readlane(m, 0));
    m = max(max(m, __builtin_amdgcn_readlane(m, 16)), max(__builtin_amdgcn_readlane(m, 32), __builtin_amdgcn_readlane(m, 48)));
    if (tid == 0) s_sink_max = m;
  }

  // ---- scoring ----------------------------------------------------------------
  uint64_t best_nearest = ~0ull;
  auto score_batch = [&](int p0, int buf) {
    // Queries two at a time, held in registers across the batch's passes (one
    // LDS read of each query slice per batch); q_s rows beyond G are read but
    // never selected into `best`.  Pinned order per (row, query) as above.
    float best[PB];
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) best[pb] = NEG_INF;
#pragma unroll 1
    for (int g = 0; g < G; g += 2) {
      float qa[16], qb[16];
      load_q_pair(q_s, g, lane8, qa, qb);
#pragma unroll
      for (int pb = 0; pb < PB; ++pb) {
        float cv[16];
        decode_frag<CT>(frag[buf][pb], cv);
        float a0, a1;
        dot16_pair<CT, DT>(qa, qb, cv, a0, a1);
        best[pb] = fmax_exact(best[pb], a0);
        if (g + 1 < G) best[pb] = fmax_exact(best[pb], a1);
      }
    }
#pragma unroll
    for (int pb = 0; pb < PB; ++pb) {
      const int c = (p0 + pb) * ROWS_PER_PASS + sub;
      const bool live = c < count && rsize[buf][pb] > 0;
      if (lane8 == 0 && c < nscore) key16[c] = f16_bits_hw(live ? best[pb] : NEG_INF);
      if (nearest_mode) {
        float cv[16];
        decode_frag<CT>(frag[buf][pb], cv);
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
        if (live) {
          const uint64_t cand = ((uint64_t)ckv_f2u(acc) << 32) | (uint32_t)c;
          best_nearest = cand < best_nearest ? cand : best_nearest;
        }
      }
    }
  };
  // Passes past the live communities (score headroom for communities that
  // have not formed yet) are skipped.  Prefetches past them are clamped to the
  // last live row (cache hits): the first use of any earlier load after the
  // loop waits for every load issued in it.
  const int live_passes = (count + ROWS_PER_PASS - 1) / ROWS_PER_PASS;
  const int last_live = max(count, 1) - 1;
  bool score_all = !PRE;
  if constexpr (COOP) {
    uint32_t need = 0;
    if (chain_wave) {
      // ---- graph-indexed chain into LDS (no barrier until the polls end) ----
      const int ct = tid - COOP_SCORE_WAVES * 64;
      constexpr int CN = SELECT_THREADS - COOP_SCORE_WAVES * 64;
      const int cp = (C + 7) & ~7;
      int* f_lo = fused_fields(dyn, C) + 2 * cp;
      int* f_dc = f_lo + cp;
      int* f_tl = f_dc + cp;
      int* f_ts = f_tl + cp;
      int* f_tn = f_ts + cp;
      hist[ct] = 0;
      hist[ct + CN] = 0;
      hist2[ct] = 0;
      hist2[ct + CN] = 0;
      fused_marks(dyn, C)[ct] = -1;  // FUSED_TILES * TILE == CN marks
      if (ct == 0) {
        s_max_idx = -1;
        s_sel_count = 0;
      }
      // Every load below is unconditional (clamped indices; dummy address when
      // there are no sinks): a branch around a load would make the next
      // round's address wait also cover the loads issued before it.
      // sinks: the first chain wave holds up to 256 positions and their maximum
      int sv[CKV_MAX_SINKS / 64];
      {
        const int32_t* sp = ns > 0 ? a.cfg.sink_positions : a.st.community_counts + rh;
#pragma unroll
        for (int i = 0; i < CKV_MAX_SINKS / 64; ++i) sv[i] = gload_i32(sp + max(min(ct + 64 * i, ns - 1), 0));
      }
      // R1: every scored row's CSR start, delta count and tail chunk, then the current position
      constexpr int CJ = OWN * SELECT_THREADS / CN;  // rows per chain thread (nscore <= OWN * SELECT_THREADS)
      int lo[CJ], dc[CJ], tl[CJ];
#pragma unroll
      for (int i = 0; i < CJ; ++i) {
        const int c = min(ct + i * CN, C - 1);
        lo[i] = gload_i32(a.csr.member_offsets + (int64_t)graph * (C + 1) + c);
        dc[i] = gload_i32(a.dl.community_sizes + (int64_t)graph * C + c);
        tl[i] = gload_i32(a.dl.community_tail + (int64_t)graph * C + c);
      }
      CKV_STAMP_AT(rh == 0 && part == 0 && ct == 0 && graph >= 0, 15);
      const int cur_g = a.st.current_position[graph];
      // R2: tail chunk start and fill, the window tokens' communities, the current key
      int ts[CJ], tn[CJ];
      const int64_t cbase = (int64_t)graph * cpg;
      CKV_STAMP_AT(rh == 0 && part == 0 && ct == 0 && tl[0] > -2, 23);
      const int cpg1 = max(cpg, 1);
      const int32_t* cstart = cpg > 0 ? a.dl.chunk_start : a.st.community_counts + rh;
      const int32_t* csz = cpg > 0 ? a.dl.chunk_size : a.st.community_counts + rh;
#pragma unroll
      for (int i = 0; i < CJ; ++i) {
        const int t = cpg > 0 ? min(max(tl[i], 0), cpg1 - 1) : 0;
        ts[i] = gload_i32(cstart + (cpg > 0 ? cbase + t : 0));
        tn[i] = gload_i32(csz + (cpg > 0 ? cbase + t : 0));
      }
      constexpr int WJ = CKV_MAX_WINDOW / CN;
      int wc[WJ];
      const int32_t* tcomm = a.st.token_communities + (int64_t)graph * a.st.token_capacity;
#pragma unroll
      for (int h = 0; h < WJ; ++h) {
        // (entries past the window are clamped to its first token: same lines)
        int64_t p = (int64_t)cur_g - W + ct + h * CN;
        p = h * CN < W ? p : (int64_t)cur_g - W;
        wc[h] = gload_i32(tcomm + (p < 0 ? 0 : (p >= a.st.token_capacity ? a.st.token_capacity - 1 : p)));
      }
      // the current key (nearest-centroid assignment only: its row is in the
      // KV cache, a page this round would otherwise not touch); issued last, so
      // the branch around it delays no other wait
      float kv_cur = 0.0f;
      if (nearest_mode) {
        const int64_t pc = cur_g < 0 ? 0 : (cur_g >= a.kv.capacity ? a.kv.capacity - 1 : cur_g);
        kv_cur = load_elem<DT>(a.kv.key, kvh * a.kv.head_stride + pc * a.kv.token_stride + ct);
      }
      if (ct < 64) {
        int m = -1;
#pragma unroll
        for (int i = 0; i < CKV_MAX_SINKS / 64; ++i) {
          if (ct + 64 * i < ns) {
            sink_s[ct + 64 * i] = sv[i];
            m = max(m, sv[i]);
          }
        }
        m = wave_max_i32(m);
        if (ct == 0) s_sink_max = m;
      }
#pragma unroll
      for (int i = 0; i < CJ; ++i) {
        const int c = ct + i * CN;
        if (c < nscore) {
          const bool alive = c < count;
          const bool has = alive && dc[i] > 0 && tl[i] >= 0 && tl[i] < cpg;
          f_lo[c] = alive ? lo[i] : 0;
          f_dc[c] = alive ? dc[i] : 0;
          f_tl[c] = alive ? tl[i] : -1;
          f_ts[c] = has ? ts[i] : 0;
          f_tn[c] = has ? tn[i] : 0;
        }
      }
#pragma unroll
      for (int h = 0; h < WJ; ++h) {
        if (ct + h * CN < W) slot_lds[ct + h * CN] = wc[h];
      }
      if (nearest_mode) key_s[ct] = (cur_g >= 0 && cur_g < a.kv.capacity) ? kv_cur : 0.0f;
      if (ct == 0) s_cur = cur_g;
#ifdef CKV_PHASE_TIMING
      if (rh == 0 && part == 0 && ts[0] > -2) atomicMax(&phase_stamp[28], (unsigned long long)wall_clock64());
#endif
    } else {
      // ---- this part's rows, published as (epoch + 1) << 32 | fp16 bits ------
      // The query-pair groups' maxima are combined lower group first, so the
      // result equals the sequential maximum over the group's queries (for
      // every non-NaN score).
      const int st_ = tid;  // scoring thread (waves 0 .. COOP_SCORE_WAVES - 1)
      if (ri == 0) {  // the query group in LDS for the fallback scoring
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int g = 2 * qp + (2 << qps_log) * j + u;
            if (g < G) {
#pragma unroll
              for (int e = 0; e < 16; ++e) {
                const uint4 w = qraw[j][u][e >> 3];
                const uint32_t x = (e & 7) < 2 ? w.x : (e & 7) < 4 ? w.y : (e & 7) < 6 ? w.z : w.w;
                q_s[g * D + 16 * lane8 + e] = ckv_u2f((e & 1) ? (x & 0xffff0000u) : (x << 16));
              }
            }
          }
        }
      }
      const int npass = (rpp + rows_pass - 1) / rows_pass;
      for (int ps = 0; ps < npass; ++ps) {
        const int i0 = ps * rows_pass;
        if (part + parts * i0 >= count) break;  // no live row in this pass or later ones (uniform)
        CentroidFrag<CT> f;
        int fsize = 0;
        const int i = i0 + ri;
        const int row = part + parts * min(i, rpp - 1);
        if (ps < COOP_PRE) {
#pragma unroll
          for (int k = 0; k < COOP_PRE; ++k) {
            if (k == ps) {
              f = cfrag[k];
              fsize = csize[k];
            }
          }
        } else {
          load_frag<CT>(a.st.centroids, (int64_t)rh * C + min(row, nscore - 1), 16 * lane8, f);
          fsize = gload_i32(a.st.community_sizes + (int64_t)rh * C + min(row, nscore - 1));
        }
        float cv[16];
        decode_frag<CT>(f, cv);
        float best = NEG_INF;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int g = 2 * qp + (2 << qps_log) * j;
          if (g < G) {
            float qa[16], qb[16];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const uint4 wa = qraw[j][0][e >> 3], wb = qraw[j][1][e >> 3];
              const int w4 = (e & 7) >> 1;
              const uint32_t xa = w4 == 0 ? wa.x : w4 == 1 ? wa.y : w4 == 2 ? wa.z : wa.w;
              const uint32_t xb = w4 == 0 ? wb.x : w4 == 1 ? wb.y : w4 == 2 ? wb.z : wb.w;
              qa[e] = ckv_u2f((e & 1) ? (xa & 0xffff0000u) : (xa << 16));
              qb[e] = ckv_u2f((e & 1) ? (xb & 0xffff0000u) : (xb << 16));
            }
            float a0, a1;
            dot16_pair<CT, DT>(qa, qb, cv, a0, a1);
            best = fmax_exact(best, a0);
            if (g + 1 < G) best = fmax_exact(best, a1);
          }
        }
        if (qps_log >= 1) best = fmax_exact(best, xor_f32<8>(best));
        const bool in = i < rpp && row < count;
        const bool live = in && fsize > 0;
        const uint16_t bits = f16_bits_hw(live ? best : NEG_INF);
        if (lane8 == 0 && qp == 0 && in) {
          key16[row] = bits;
          if (xcd_local) st_xcd_u64(xrow + row, tag | bits); else st_agent_u64(xrow + row, tag | bits);
        }
      }
      CKV_TS(14);
      CKV_STAMP_MAX(rh == 0, 27);
      {
        // Each scoring thread polls the other parts' rows among its rows st_,
        // st_ + 384, ... until every one carries this launch's tag (a wave
        // leaves once all its rows have arrived; bounded: a part that still
        // misses rows scores every community itself).  One tagged word per
        // row, so a row is taken as soon as its own store lands, without a
        // per-part completion word and the second round it would need.
        constexpr int SN = COOP_SCORE_WAVES * 64;
        constexpr int PJ = (OWN * SELECT_THREADS + SN - 1) / SN;
#pragma unroll
        for (int k = 0; k < PJ; ++k) {
          const int c = st_ + k * SN;
          if (c < count && c % parts != part) need |= 1u << k;
        }
        for (int pr = 0; pr < COOP_POLLS && __ballot(need != 0) != 0ull; ++pr) {
          uint64_t v[PJ];
#pragma unroll
          for (int k = 0; k < PJ; ++k) v[k] = ld_agent_u64(xrow + min(st_ + k * SN, C - 1));
#pragma unroll
          for (int k = 0; k < PJ; ++k) {
            if (((need >> k) & 1u) && (v[k] & 0xffffffff00000000ull) == tag) {
              key16[st_ + k * SN] = (uint16_t)v[k];
              need &= ~(1u << k);
            }
          }
          if (__ballot(need != 0) != 0ull) __builtin_amdgcn_s_sleep(4);
        }
      }
    }
    CKV_STAMP_AT(rh == 0 && part == 0 && tid == 0, 13);
    score_all = __syncthreads_or(need != 0);  // key16 complete (or fallback), chain fields in LDS
    cur = s_cur;
    if (nearest_mode) {
      // squared distance of the current key to this part's live rows (scoring
      // waves; the fragments are still in registers), one minimum per wave of
      // every part, tagged with the epoch's low 16 bits:
      // distance bits << 32 | row << 16 | tag
      uint64_t best_share = ~0ull;
      if (!chain_wave) {
        const int npass = (rpp + rows_pass - 1) / rows_pass;
        for (int ps = 0; ps < npass; ++ps) {
          const int i0 = ps * rows_pass;
          if (part + parts * i0 >= count) break;
          CentroidFrag<CT> f;
          int fsize = 0;
          const int i = i0 + ri;
          const int row = part + parts * min(i, rpp - 1);
          if (ps < COOP_PRE) {
#pragma unroll
            for (int k = 0; k < COOP_PRE; ++k) {
              if (k == ps) {
                f = cfrag[k];
                fsize = csize[k];
              }
            }
          } else {
            load_frag<CT>(a.st.centroids, (int64_t)rh * C + min(row, nscore - 1), 16 * lane8, f);
            fsize = gload_i32(a.st.community_sizes + (int64_t)rh * C + min(row, nscore - 1));
          }
          float cv[16];
          decode_frag<CT>(f, cv);
          float acc;
          {
            const float d0 = key_s[16 * lane8] - cv[0];
            acc = d0 * d0;
          }
#pragma unroll
          for (int e = 1; e < 16; ++e) {
            const float di = key_s[16 * lane8 + e] - cv[e];
            acc = acc + di * di;
          }
          acc = add_xor_f32<4>(acc);
          acc = add_xor_f32<2>(acc);
          acc = add_xor_f32<1>(acc);
          if (i < rpp && row < count && fsize > 0 && qp == 0) {
            const uint64_t cand = ((uint64_t)ckv_f2u(acc) << 32) | ((uint64_t)(uint32_t)row << 16);
            best_share = cand < best_share ? cand : best_share;
          }
        }
      }
      const uint64_t w = wave_min_u64(best_share);
      if ((tid & 63) == 0) st_agent_u64(xrow + C + part * WAVES + (tid >> 6), (w | 0xffffull) ^ 0xffffull ^ near_tag16(epoch));
    }
  }
  if constexpr (PRE) {
#pragma unroll
    for (int k = 0; k < OWN; ++k) {
      const int c = tid + k * SELECT_THREADS;
      if (c < count) key16[c] = pre_key[k];
    }
  } else if (score_all) {
    if constexpr (COOP) {  // fallback: every community scored here
      load_batch(0, 0, nscore - 1);
      load_batch(PB, 1, nscore - 1);
    }
    for (int p0 = 0; p0 < live_passes; p0 += 2 * PB) {
      score_batch(p0, 0);
      if (p0 + PB >= live_passes) break;
      load_batch(p0 + 2 * PB, 0, last_live);
      score_batch(p0 + PB, 1);
      load_batch(p0 + 3 * PB, 1, last_live);
    }
  }
  CKV_TS(7);
  if (nearest_mode) {
    const uint64_t w = wave_min_u64(best_nearest);
    if ((tid & 63) == 0) near_s[tid >> 6] = w;
  }
  __syncthreads();  // key16, near_s
  CKV_TS(1);

  // ---- R2: tail-chunk fields; communities of the window tokens ---------------
  // Issued after the scoring: their addresses need the R1 fields and the
  // current position, and nothing before the compaction reads them, so the
  // scoring starts as soon as the R0 data is in.  Every earlier load has
  // landed by now (the R1 fields long ago, the last prefetches are cache
  // hits); waiting for them here keeps the waits for older loads after the
  // conditional R2 issue from also waiting for R2.
  if constexpr (!COOP || CKV_R2_LATE) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    issue_r2();
  }
  // masks of the R0/R1 fields (R2 fields stay raw until used: masking them here would wait for R2)
#pragma unroll
  for (int k = 0; k < OWN; ++k) {
    const int c = cid(k);
    if (c >= nscore) o_size[k] = 0;
    if (c >= count) {
      o_lo[k] = 0;
      o_dc[k] = 0;
      o_tl[k] = -1;
    }
  }
  // ---- exact weighted selection ---------------------------------------------
  const bool budget_mode = a.cfg.selection_mode == CKV_SELECT_BUDGET;
  const int sel_slots = a.cfg.max_selected;
  const int target = budget_mode ? sel_slots : a.cfg.topk_communities;
  uint32_t o_key[OWN];
#pragma unroll
  for (int k = 0; k < OWN; ++k) {
    const int c = cid(k);
    const bool live = c < count && o_size[k] > 0;
    o_key[k] = live ? ckv_ordered_key16(key16[c]) : 0u;
    if (live) atomicAdd(hist + (o_key[k] >> 8), budget_mode ? o_size[k] : 1);
  }
  __syncthreads();
  CKV_TS(12);
  // key16 is dead from here on (unfused); it becomes the community -> descriptor table.
  uint16_t* comm_desc = key16;
  if constexpr (!FUSED) {
    for (int c = tid; c < nscore; c += SELECT_THREADS) comm_desc[c] = 0xffffu;
  }
  // Every wave finds the bins itself (same histogram, same result): no
  // barrier to broadcast them.
  int hb, above_hb;
  wave_find_bin(hist, target, hb, above_hb);
  int threshold;  // 16-bit key threshold; -1 selects every non-empty community
  if (hb < 0) {
    threshold = -1;
  } else {
#pragma unroll
    for (int k = 0; k < OWN; ++k) {
      const int c = cid(k);
      const bool live = c < count && o_size[k] > 0;
      if (live && (int)(o_key[k] >> 8) == hb) atomicAdd(hist2 + (o_key[k] & 0xff), budget_mode ? o_size[k] : 1);
    }
    __syncthreads();
    int lb, above_lb;
    wave_find_bin(hist2, target - above_hb, lb, above_lb);
    threshold = (hb << 8) | lb;
  }
  CKV_TS(2);

  // Compaction, high keys first (id order), then threshold keys (id order): one
  // four-component block scan (high count/mass, threshold count/mass).
  const int cap_tokens = sel_slots;
  // One scan per ownership round k (the rounds are consecutive id ranges).
  int b4k[OWN][4], t4[4] = {0, 0, 0, 0};
  {
    const int lane = tid & 63, wave = tid >> 6;
    int v4[OWN][4], inc[OWN][4];
#pragma unroll
    for (int k = 0; k < OWN; ++k) {
      const int c = cid(k);
      const int size = o_size[k];
      const bool ok = c < count && size > 0;
      const bool high = ok && (int)o_key[k] > threshold;
      const bool eq = ok && threshold >= 0 && (int)o_key[k] == threshold;
      v4[k][0] = high ? 1 : 0;
      v4[k][1] = high ? size : 0;
      v4[k][2] = eq ? 1 : 0;
      v4[k][3] = eq ? size : 0;
      if (k > 0 && k * SELECT_THREADS >= count) {  // a round without live communities (uniform)
#pragma unroll
        for (int i = 0; i < 4; ++i) inc[k][i] = 0;
        continue;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) inc[k][i] = wave_inclusive_scan(v4[k][i]);
      if (lane == 63)
        *reinterpret_cast<int4*>(scan_s + 4 * (k * WAVES + wave)) = int4{inc[k][0], inc[k][1], inc[k][2], inc[k][3]};
    }
    CKV_TS(8);
    __syncthreads();
    CKV_TS(9);
#pragma unroll
    for (int k = 0; k < OWN; ++k) {
#pragma unroll
      for (int i = 0; i < 4; ++i) b4k[k][i] = inc[k][i] - v4[k][i] + t4[i];
      if (k > 0 && k * SELECT_THREADS >= count) continue;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const int4 x = *reinterpret_cast<const int4*>(scan_s + 4 * (k * WAVES + w));
        const int xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (w < wave) b4k[k][i] += xs[i];
          t4[i] += xs[i];
        }
      }
    }
  }
  const int high_count = t4[0], high_mass = t4[1];
  const int cap_sel = sel_slots;
  int fused_pos = -1;  // FUSED: this lane's slot of its wave's tile
  if constexpr (FUSED) {
    // ---- fused slot resolution --------------------------------------------
    // Each owner thread places its selected community: its selection start
    // and membership fields go to LDS by community id, and a mark at the
    // first slot it covers in each of this part's tiles, so a tile lane finds
    // its community with one ballot (no descriptor search), and it writes its
    // own descriptor and tile-descriptor outputs.  The window slots look their
    // token's community up by id; the truncated last community's oldest
    // attended member is gathered by the window lanes that need it, in the
    // same round as the members (no workgroup barrier in between).
    const int cp = (C + 7) & ~7;
    int* f_st = fused_fields(dyn, C);  // selection start of each community, -1 when not selected
    int* f_size = f_st + cp;
    int* f_lo = f_size + cp;
    int* f_dc = f_lo + cp;
    int* f_tl = f_dc + cp;
    int* f_ts = f_tl + cp;
    int* f_tn = f_ts + cp;
    int* f_idx = f_tn + cp;  // descriptor index of each selected community
    int* marks = fused_marks(dyn, C);
    int* td_s = marks + FUSED_TILES * TILE;  // this part's tile descriptors (tiles part, part + parts, ...)
    const int dcap_ = a.ws.descriptor_capacity;
    int my_max = -1, my_end = 0;
#pragma unroll
    for (int k = 0; k < OWN; ++k) {
      const int c = cid(k);
      int hc = b4k[k][0], hm = b4k[k][1], ec = b4k[k][2], em = b4k[k][3];
      const int size = o_size[k];
      const bool ok = c < count && size > 0;
      const bool high = ok && (int)o_key[k] > threshold;
      const bool eq = ok && threshold >= 0 && (int)o_key[k] == threshold;
      int st = -1, en = 0, idx = -1;
      if (high) {
        if (hm < cap_sel && hc < dcap_) {
          st = hm;
          en = min(cap_sel, hm + size);
          idx = hc;
        }
        hc += 1;
        hm += size;
      } else if (eq) {
        const int st0 = high_mass + em;
        const bool within = budget_mode ? (st0 < sel_slots) : (ec < a.cfg.topk_communities - high_count);
        const int i2 = high_count + ec;
        if (within && st0 < cap_sel && i2 < dcap_) {
          st = st0;
          en = min(cap_sel, st0 + size);
          idx = i2;
        }
        ec += 1;
        em += size;
      }
      if (c < cp) f_st[c] = st;
      if (st >= 0) {
        f_idx[c] = idx;
        f_size[c] = size;
        if constexpr (!COOP) {  // (COOP: written by the chain waves)
          f_lo[c] = o_lo[k];
          f_dc[c] = o_dc[k];
          f_tl[c] = o_tl[k];
          const bool has = o_dc[k] > 0 && o_tl[k] >= 0 && o_tl[k] < cpg;
          f_ts[c] = has ? o_ts[k] : 0;
          f_tn[c] = has ? o_tn[k] : 0;
        }
#pragma unroll
        for (int w = 0; w < FUSED_TILES; ++w) {
          const int t0 = (part * FUSED_TILES + w) * TILE - ns;
          if (st < t0 + TILE && en > t0) marks[w * TILE + max(st, t0) - t0] = c;
        }
        my_max = max(my_max, idx);
        my_end = max(my_end, en);
        // this part's tile descriptors whose first selected slot lies here
        // (LDS only: a global store here would make the tile waves' later
        // memory waits cover it)
        for (int t = part, q = 0; t < a.ws.budget_tiles; t += parts, ++q) {
          const int off = max(t * TILE - ns, 0);
          if (st <= off && off < en) td_s[q] = idx;
        }
      }
    }
    CKV_TS(16);
    {  // totals: one DPP maximum per wave, then one LDS atomic per wave
      const int wmax = wave_max_i32(my_max);
      const int wend = wave_max_i32(my_end);
      if ((tid & 63) == 0 && wmax >= 0) {
        atomicMax(&s_max_idx, wmax);
        atomicMax(&s_sel_count, wend);
      }
    }
    if constexpr (!COOP) {
#pragma unroll
      for (int h = 0; h < WIN_PER_THREAD; ++h) {
        const int i = tid + h * SELECT_THREADS;
        if (i < W) slot_lds[i] = wcomm[h];
      }
    }
    CKV_TS(10);
    __syncthreads();  // fields, marks, totals, window communities
    CKV_TS(3);
    const int n_desc = s_max_idx + 1;
    const int sel_count = s_sel_count;
    const int lane = tid & 63, wave = tid >> 6;
    if (wave < FUSED_TILES) {
      const int slot_cap = a.ws.slot_capacity;
      const int tile = part * FUSED_TILES + wave;
      const int s = tile * TILE + lane;
      const int j = s - ns;
      const int wbeg = ns + sel_count;
      const int inc = a.cfg.include_current ? 1 : 0;
      const int32_t* members = a.csr.member_positions + (int64_t)graph * a.csr.member_stride;
      const int32_t* dpos = a.dl.positions + (int64_t)graph * a.dl.position_capacity;
      const int mk = marks[wave * TILE + lane];
      const uint64_t mm = __ballot(mk >= 0);
      const int32_t* src = a.st.community_counts + rh;  // in-bounds dummy address when nothing is gathered
      bool gathered = false;
      int slow_c = -1, slow_rem = 0;
      // member m (newest first) of community c: a tail-chunk delta, a CSR
      // member, or (slow_c >= 0) a delta member older than the tail chunk
      auto member_src_c = [&](int c, int m) {
        const int dc = f_dc[c];
        if (m < dc) {
          const int tn = f_tn[c];
          if (m < tn) {
            const int p = f_ts[c] + tn - 1 - m;
            if (p >= 0 && p < a.dl.position_capacity) {
              src = dpos + p;
              gathered = true;
            }
          } else {
            slow_c = c;
            slow_rem = m - tn;
          }
        } else {
          const int64_t idx = (int64_t)f_lo[c] + (m - dc);
          if (idx >= 0 && idx < a.csr.member_stride) {
            src = members + idx;
            gathered = true;
          }
        }
      };
      int kind = 0;  // 1 sink, 2 selected member, 3 window, 4 current
      int wpos = -1;
      bool need_last = false;
      if (tile < slot_cap / TILE) {
        if (s < ns) {
          kind = 1;
        } else if (j < sel_count) {
          kind = 2;
          const uint64_t upto = mm & (lane == 63 ? ~0ull : ((2ull << lane) - 1ull));
          if (upto != 0) {  // always: the community covering a selected slot marks it or an earlier one
            const int c = marks[wave * TILE + 63 - __builtin_clzll(upto)];
            member_src_c(c, j - f_st[c]);
          }
        } else if (s < wbeg + W) {
          kind = 3;
          const int i = s - wbeg;
          const int p = cur - W + i;
          wpos = p < 0 ? -1 : p;
          if (wpos >= 0 && p <= s_sink_max) {
            for (int q = 0; q < ns; ++q) {
              if (sink_s[q] == p) wpos = -1;
            }
          }
          const int wc = slot_lds[i];
          if (wpos >= 0 && p < a.st.token_capacity && wc >= 0 && wc < count && f_st[wc] >= 0) {
            const int take = min(f_size[wc], cap_sel - f_st[wc]);
            if (take >= f_size[wc]) {
              wpos = -1;  // the whole community is attended already
            } else {
              // the truncated last community: attended already when at or
              // after its oldest attended member
              need_last = true;
              member_src_c(wc, take - 1);
            }
          }
        } else if (inc && s == wbeg + W) {
          kind = 4;
        }
      }
      CKV_TS(17);
      int val = gload_i32(src);
      if (!gathered) val = -1;
      if (slow_c >= 0) {
        val = -1;
        const int tail = f_tl[slow_c];
        if (tail >= 0 && tail < cpg) {
          int rem = slow_rem;
          int ch = a.dl.chunk_previous[cb + tail];
          for (int guard = 0; guard < 64 && ch >= 0 && ch < cpg; ++guard) {
            const int cs = a.dl.chunk_size[cb + ch];
            if (rem < cs) {
              const int p = a.dl.chunk_start[cb + ch] + cs - 1 - rem;
              if (p >= 0 && p < a.dl.position_capacity) val = dpos[p];
              break;
            }
            rem -= cs;
            ch = a.dl.chunk_previous[cb + ch];
          }
        }
      }
      if (kind == 1) fused_pos = sink_s[s];
      else if (kind == 2) fused_pos = val;
      else if (kind == 3) fused_pos = (need_last && wpos >= val) ? -1 : wpos;
      else if (kind == 4) fused_pos = cur;
      CKV_TS(4);
    } else {
      // ---- this part's share of the selection outputs (waves without a tile) ----
      const int ot = tid - FUSED_TILES * 64;
      const int on = SELECT_THREADS - FUSED_TILES * 64;
      if (part == 0 && ot == 0) {
        a.ws.descriptor_counts[rh] = n_desc;
        a.ws.selected_counts[rh] = sel_count;
      }
      for (int c = part + parts * ot; c < nscore; c += parts * on) {
        const int st = c < count ? f_st[c] : -1;
        if (st >= 0) {
          const int idx = f_idx[c];
          a.ws.communities[(int64_t)rh * dcap_ + idx] = c;
          a.ws.cumulative_ends[(int64_t)rh * dcap_ + idx] = min(cap_sel, st + f_size[c]);
        }
        a.ws.scores[(int64_t)rh * C + c] = c < count ? key16[c] : (uint16_t)0xfc00u;
      }
      for (int t = part + parts * ot, q = ot; t < a.ws.budget_tiles; t += parts * on, q += on) {
        const int off = max(t * TILE - ns, 0);
        a.ws.tile_descriptors[(int64_t)rh * a.ws.budget_tiles + t] = off < sel_count ? td_s[q] : max(0, n_desc - 1);
      }
      if (nearest_mode && !COOP && tid == FUSED_TILES * 64 && part == parts - 1) {
        uint64_t m = ~0ull;
        for (int w = 0; w < WAVES; ++w) m = near_s[w] < m ? near_s[w] : m;
        a.ws.nearest[rh] = (m == ~0ull) ? -1 : (int)(m & 0xffffffffu);
      }
    }
  } else {
  // Also marks idx as the first descriptor of every 64-slot block whose first
    // slot falls in [start, end) (the ranges partition the selection).
    auto store_desc = [&](int idx, int c, int start, int end, int k) {
      desc_comm[idx] = c;
      desc_end[idx] = end;
      for (int b = (start + 63) >> 6; (b << 6) < end; ++b) blk_first[b] = idx;
      desc_lo[idx] = o_lo[k];
      desc_dc[idx] = o_dc[k];
      desc_tl[idx] = o_tl[k];
      const bool has = o_dc[k] > 0 && o_tl[k] >= 0 && o_tl[k] < cpg;
      desc_ts[idx] = has ? o_ts[k] : 0;
      desc_tn[idx] = has ? o_tn[k] : 0;
    };
    {
        int my_max = -1;
  #pragma unroll
      for (int k = 0; k < OWN; ++k) {
        const int c = cid(k);
        int hc = b4k[k][0], hm = b4k[k][1], ec = b4k[k][2], em = b4k[k][3];
        const int size = o_size[k];
        const bool ok = c < count && size > 0;
        const bool high = ok && (int)o_key[k] > threshold;
        const bool eq = ok && threshold >= 0 && (int)o_key[k] == threshold;
        if (high) {
          if (hm < cap_tokens && hc < dcap) {
            store_desc(hc, c, hm, min(cap_tokens, hm + size), k);
            my_max = max(my_max, hc);  // (a later high-key community has a smaller index than an earlier threshold one)
          }
          hc += 1;
          hm += size;
        } else if (eq) {
          const int st0 = high_mass + em;
          const bool within = budget_mode ? (st0 < sel_slots) : (ec < a.cfg.topk_communities - high_count);
          const int idx = high_count + ec;
          if (within && st0 < cap_tokens && idx < dcap) {
            store_desc(idx, c, st0, min(cap_tokens, st0 + size), k);
            my_max = max(my_max, idx);
          }
          ec += 1;
          em += size;
        }
      }
      CKV_TS(10);
      const int wmax = wave_max_i32(my_max);  // one LDS atomic per wave
      if ((tid & 63) == 0 && wmax >= 0) atomicMax(&s_max_idx, wmax);
    }
    __syncthreads();  // descriptors, s_max_idx
    const int n_desc = s_max_idx + 1;
    const int sel_count = n_desc > 0 ? desc_end[n_desc - 1] : 0;
    CKV_TS(15);
    if (tid == 0) blk_first[(sel_count + 63) / 64] = n_desc;  // (blocks below were marked by store_desc)
    for (int d = tid; d < n_desc; d += SELECT_THREADS) comm_desc[desc_comm[d]] = (uint16_t)d;
    // Only the last descriptor can be truncated; remember its community size.
    if (n_desc > 0) {
      const int last_c = desc_comm[n_desc - 1];
      if (last_c % SELECT_THREADS == tid) {
  #pragma unroll
        for (int k = 0; k < OWN; ++k) {
          if (cid(k) == last_c) s_last_size = o_size[k];
        }
      }
    }
    if (tid == 0) s_last_sel_pos = -1;
    CKV_TS(3);
  
    const int slot_cap = a.ws.slot_capacity;
    int32_t* slots = a.ws.slot_positions + (int64_t)rh * slot_cap;
    const int inc = a.cfg.include_current ? 1 : 0;
    const int wbeg = ns + sel_count;
    if (materialise) {
      __syncthreads();  // blk_first, comm_desc, s_last_size
      CKV_TS(16);
      // ---- R3: slot materialisation ---------------------------------------------
      // Layout: sinks, selected members (newest first: decode deltas from the
      // tail chunk backwards, then the recency-descending CSR), window, current.
      const int32_t* members = a.csr.member_positions + (int64_t)graph * a.csr.member_stride;
      const int32_t* dpos = a.dl.positions + (int64_t)graph * a.dl.position_capacity;
      const int lane = tid & 63, wave = tid >> 6;
      // Source of selected member j (0 <= j < sel_count) of descriptor d: a
      // decode-delta position of the tail chunk, a CSR member, or (slow_d >= 0) a
      // delta member older than the tail chunk, resolved by walk_chain.
      auto member_src = [&](int j, int d, const int32_t*& src, bool& gathered, int& slow_d, int& slow_rem) {
        const int m = j - (d > 0 ? desc_end[d - 1] : 0);
        const int dc = desc_dc[d];
        if (m < dc) {
          const int tn = desc_tn[d];
          if (m < tn) {
            const int p = desc_ts[d] + tn - 1 - m;
            if (p >= 0 && p < a.dl.position_capacity) {
              src = dpos + p;
              gathered = true;
            }
          } else {
            slow_d = d;
            slow_rem = m - tn;
          }
        } else {
          const int64_t idx = (int64_t)desc_lo[d] + (m - dc);
          if (idx >= 0 && idx < a.csr.member_stride) {
            src = members + idx;
            gathered = true;
          }
        }
      };
      auto walk_chain = [&](int d, int rem, int& val) {
        const int tail = desc_tl[d];
        if (tail < 0 || tail >= cpg) return;
        int ch = a.dl.chunk_previous[cb + tail];
        for (int guard = 0; guard < 64 && ch >= 0 && ch < cpg; ++guard) {
          const int cs = a.dl.chunk_size[cb + ch];
          if (rem < cs) {
            const int p = a.dl.chunk_start[cb + ch] + cs - 1 - rem;
            if (p >= 0 && p < a.dl.position_capacity) val = dpos[p];
            return;
          }
          rem -= cs;
          ch = a.dl.chunk_previous[cb + ch];
        }
      };
      // Window slot i (position cur-W+i), or -1 when that token is already
      // attended (a sink, or a member of a selected community at or after the
      // selection's oldest position); wc is the token's community.
      auto window_pos = [&](int i, int wc, int last_pos) {
        const int p = cur - W + i;
        int pos = p < 0 ? -1 : p;
        if (pos >= 0 && p <= s_sink_max) {
          for (int k = 0; k < ns; ++k) {
            if (sink_s[k] == p) pos = -1;
          }
        }
        if (pos >= 0 && p < a.st.token_capacity && wc >= 0 && wc < count) {
          const int found = comm_desc[wc] == 0xffffu ? -1 : (int)comm_desc[wc];
          if (found >= 0) {
            const int take = desc_end[found] - (found > 0 ? desc_end[found - 1] : 0);
            const bool full = found < n_desc - 1 || take >= s_last_size;
            if (full || p >= last_pos) pos = -1;
          }
        }
        return pos;
      };
      {
        // Each wave resolves 64-slot blocks of the selection, lane = slot
        // (coalesced gathers): a lane's descriptor is the block's first descriptor
        // plus the number of descriptor ends at or before it, read off a wave-wide
        // bit mask of the ends that fall inside the block (no search chains).
        // (parts > 1: this workgroup resolves the blocks b with b % parts == part;
        // every part ran the same selection)
        const int nblk_sel = (sel_count + 63) / 64;
        const int nblk_own = nblk_sel > part ? (nblk_sel - part + parts - 1) / parts : 0;
        for (int b0 = wave; b0 < nblk_own; b0 += WAVES * MAT_BATCH) {
          const int32_t* src[MAT_BATCH];
          bool gathered[MAT_BATCH];
          int slow_d[MAT_BATCH], slow_rem[MAT_BATCH];
  #pragma unroll
          for (int q = 0; q < MAT_BATCH; ++q) {
            const int b = part + parts * (b0 + q * WAVES);
            src[q] = a.st.community_counts + rh;  // in-bounds dummy address when nothing is gathered
            gathered[q] = false;
            slow_d[q] = -1;
            slow_rem[q] = 0;
            if (b < nblk_sel) {  // wave-uniform
              const int base = 64 * b;
              const int j = base + lane;
              const int d0 = blk_first[b];
              const int e = d0 + lane < n_desc ? desc_end[d0 + lane] : 0x7fffffff;
              const int off = e - base;
              const uint64_t mask = wave_or_u64(off >= 1 && off <= 63 ? (1ull << off) : 0ull);
              const uint64_t below = lane == 63 ? ~0ull : ((2ull << lane) - 1ull);
              const int d = d0 + __popcll(mask & below);
              if (j < sel_count) member_src(j, d, src[q], gathered[q], slow_d[q], slow_rem[q]);
            }
          }
          CKV_TS(17);
          int val[MAT_BATCH];
  #pragma unroll
          for (int q = 0; q < MAT_BATCH; ++q) val[q] = gload_i32(src[q]);
  #pragma unroll
          for (int q = 0; q < MAT_BATCH; ++q) {
            if (!gathered[q]) val[q] = -1;
          }
  #pragma unroll
          for (int q = 0; q < MAT_BATCH; ++q) {
            if (slow_d[q] >= 0) walk_chain(slow_d[q], slow_rem[q], val[q]);
          }
  #pragma unroll
          for (int q = 0; q < MAT_BATCH; ++q) {
            const int j = 64 * (part + parts * (b0 + q * WAVES)) + lane;
            if (j < sel_count) {
              slots[ns + j] = val[q];
              if (j == sel_count - 1) s_last_sel_pos = val[q];
            }
          }
        }
        if (tid < ns && part == 0) slots[tid] = sink_s[tid];
        __syncthreads();  // s_last_sel_pos
        CKV_TS(4);
        // the window, the current token and the padding: the part that resolved
        // the selection's last block (it knows the oldest attended member)
        if (part == (nblk_sel > 0 ? (nblk_sel - 1) % parts : 0)) {
          const int last_pos = s_last_sel_pos;
  #pragma unroll
          for (int h = 0; h < WIN_PER_THREAD; ++h) {
            const int i = tid + h * SELECT_THREADS;
            if (i < W) slots[wbeg + i] = window_pos(i, wcomm[h], last_pos);
          }
          if (inc && tid == 0) slots[wbeg + W] = cur;
          for (int s = wbeg + W + inc + tid; s < slot_cap; s += SELECT_THREADS) slots[s] = -1;
        }
      }
    }
    // ---- outputs that nothing in this kernel reads back --------------------------
    // (fused: split over the head's parts, so no part carries them all, and
    // written by the waves that attend no tile: their attention buffers lie
    // past the selection arrays, so the tile waves start attending at once)
    CKV_TS(11);
    {
      const int wp = part, wn = parts;
      const int ot = tid;
      const int stride = SELECT_THREADS;
      if (ot == 0 && wp == 0) {
        a.ws.descriptor_counts[rh] = n_desc;
        a.ws.selected_counts[rh] = sel_count;
      }
      // item i goes to part i % wn (each part writes a strided share)
      for (int i = wp + wn * ot; ot >= 0 && i < n_desc; i += stride) {
        a.ws.communities[(int64_t)rh * dcap + i] = desc_comm[i];
        a.ws.cumulative_ends[(int64_t)rh * dcap + i] = desc_end[i];
      }
      for (int t = wp + wn * ot; ot >= 0 && t < a.ws.budget_tiles; t += stride) {
        // first descriptor ending after the tile's first selected slot (searched
        // between the first descriptors of its 64-slot block and the next)
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
      if (tid % wn == wp) {
  #pragma unroll
        for (int k = 0; k < OWN; ++k) {
          const int c = cid(k);
          if (c < nscore) {
            const bool live = c < count && o_size[k] > 0;
            const uint32_t key = o_key[k];
            const uint16_t bits =
                live ? (uint16_t)((key & 0x8000u) ? (key ^ 0x8000u) : (key ^ 0xffffu)) : (uint16_t)0xfc00u;
            a.ws.scores[(int64_t)rh * C + c] = bits;
          }
        }
      }
      if (nearest_mode && !COOP && tid == 0 && wp == wn - 1) {
        uint64_t m = ~0ull;
        for (int w = 0; w < WAVES; ++w) m = near_s[w] < m ? near_s[w] : m;
        a.ws.nearest[rh] = (m == ~0ull) ? -1 : (int)(m & 0xffffffffu);
      }
    }
}
  CKV_TS(5);
  if constexpr (FUSED) {
    attend_part<SELECT_THREADS / 64, FUSED_TILES, COOP>(
        a, rh, part, parts, fused_pos, dyn + fused_select_bytes(C, a.ws.budget_tiles, parts) CKV_TS_PASS);
  }
  CKV_TS_FLUSH(rh == 0 && part == 0);
  if constexpr (COOP) coop_finish<PMAX>(a, rh, parts, epoch, nearest_mode, xrow);
}

template <int CT, int DT, int OWN>
// `parts` workgroups per head each run the selection and resolve a strided
// share of the slot blocks and outputs.
__global__ __launch_bounds__(SELECT_THREADS) void select_kernel(DecodeArgs a, DecodeArgs u, int parts) {
  const int nsel = a.st.retrieval_heads * parts;
  if ((int)blockIdx.x >= nsel) {
    const int urh = (int)blockIdx.x - nsel;
    owner_update<CT, DT>(u, urh, u.ws.lse[(int64_t)urh * u.cfg.group_size]);
    return;
  }
  select_body<CT, DT, OWN>(a, blockIdx.x % a.st.retrieval_heads, blockIdx.x / a.st.retrieval_heads, parts);
}

// Fused selection + attention partials: `parts` workgroups per retrieval head
// (workgroup w: head w / parts, part w % parts); workgroups beyond them run the
// pending online update of another layer `u`.
// PMAX > 0: cooperative scoring and the in-launch split merge (parts <= PMAX).
// Cooperative parts of a head are interleaved (head = block % heads): the
// dispatcher deals blocks to the XCDs round robin, so with 8 heads every
// part of a head shares one XCD's L2, and each head's parts span the whole
// dispatch order instead of its tail.
template <int CT, int DT, int OWN, int PMAX = 0>
__global__ __launch_bounds__(SELECT_THREADS) void select_attend_kernel(DecodeArgs a, DecodeArgs u, int parts) {
  const int nsel = a.st.retrieval_heads * parts;
  if ((int)blockIdx.x >= nsel) {
    const int urh = (int)blockIdx.x - nsel;
    owner_update<CT, DT>(u, urh, u.ws.lse[(int64_t)urh * u.cfg.group_size]);
    return;
  }
  if constexpr (PMAX > 0)
    select_body<CT, DT, OWN, true, false, true, PMAX>(a, blockIdx.x % a.st.retrieval_heads,
                                                       blockIdx.x / a.st.retrieval_heads, parts);
  else
    select_body<CT, DT, OWN, true>(a, blockIdx.x / parts, blockIdx.x % parts, parts);
}

template <int CT, int DT, int OWN>
__global__ __launch_bounds__(SELECT_THREADS) void select_attend_batch_kernel(const DecodeArgs* __restrict__ table,
                                                                            int heads, int parts) {
  const int per_item = heads * parts;
  const int r = blockIdx.x % per_item;
  select_body<CT, DT, OWN, true>(table[blockIdx.x / per_item], r / parts, r % parts, parts);
}

// Scores of 64 centroid rows of one (item, head) per workgroup, written to
// a.ws.scores as fp16 bits (-inf for empty or inactive rows), in exactly the
// selection's scoring arithmetic (dot16_pair); workgroups past the head's
// live rows exit.  Lets a batch with many communities per head score on every
// compute unit before the one-workgroup-per-head selection.
template <int CT, int DT>
__global__ __launch_bounds__(SELECT_THREADS) void score_rows_batch_kernel(const DecodeArgs* __restrict__ table,
                                                                         int heads) {
  __shared__ float q_s[CKV_MAX_GROUP * D];
  const DecodeArgs& a = table[blockIdx.y / heads];
  const int rh = blockIdx.y % heads;
  const int tid = threadIdx.x;
  const int C = a.st.community_capacity;
  const int nscore = min(C, a.ws.score_blocks * SCORE_BLOCK);
  int count = a.st.community_counts[rh];
  count = count < 0 ? 0 : (count > nscore ? nscore : count);
  const int r0 = blockIdx.x * ROWS_PER_PASS;
  if (r0 >= count) return;
  const int G = a.cfg.group_size;
  const int sub = tid >> 3, lane8 = tid & 7;
  const int row = min(r0 + sub, count - 1);
  CentroidFrag<CT> frag;
  load_frag<CT>(a.st.centroids, (int64_t)rh * C + row, 16 * lane8, frag);
  const int size = gload_i32(a.st.community_sizes + (int64_t)rh * C + row);
  for (int e = tid; e < G * D; e += SELECT_THREADS) q_s[e] = load_elem<DT>(a.kv.query, (int64_t)rh * G * D + e);
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
  if (lane8 == 0 && c < count)
    reinterpret_cast<uint16_t*>(a.ws.scores)[(int64_t)rh * C + c] = f16_bits_hw(size > 0 ? best : NEG_INF);
}

// Workgroups from `nsel` on run the pending online update of another batch
// `utable` (workgroup nsel + w: item w / uheads, head w % uheads).
template <int CT, int DT>
__device__ __forceinline__ void pending_batch_update(const DecodeArgs* __restrict__ utable, int uheads, int w) {
  const DecodeArgs& u = utable[w / uheads];
  const int urh = w % uheads;
  // nine slots per thread: a 4,096-token budget's 4,235 slots in one load round
  owner_update<CT, DT, 9>(u, urh, u.ws.lse[(int64_t)urh * u.cfg.group_size]);
}

template <int CT, int DT, int OWN>
// `parts` workgroups per (item, head) each run the selection and resolve a
// strided share of the slot table's 64-slot blocks (and of the other outputs).
__global__ __launch_bounds__(SELECT_THREADS) void select_prescored_batch_kernel(const DecodeArgs* __restrict__ table,
                                                                               int heads, int parts, int nsel,
                                                                               const DecodeArgs* __restrict__ utable,
                                                                               int uheads) {
  if ((int)blockIdx.x >= nsel) {
    pending_batch_update<CT, DT>(utable, uheads, (int)blockIdx.x - nsel);
    return;
  }
  const int per_item = heads * parts;
  const int r = blockIdx.x % per_item;
  select_body<CT, DT, OWN, false, true>(table[blockIdx.x / per_item], r % heads, r / heads, parts);
}

// Batched selection: workgroup w serves item w / heads, head w % heads of the
// device table.
template <int CT, int DT, int OWN>
__global__ __launch_bounds__(SELECT_THREADS) void select_batch_kernel(const DecodeArgs* __restrict__ table, int heads,
                                                                      int nsel, const DecodeArgs* __restrict__ utable,
                                                                      int uheads) {
  if ((int)blockIdx.x >= nsel) {
    pending_batch_update<CT, DT>(utable, uheads, (int)blockIdx.x - nsel);
    return;
  }
  select_body<CT, DT, OWN>(table[blockIdx.x / heads], blockIdx.x % heads);
}

// key16 / community table (scored rows), the descriptor arrays, the per-block descriptor index.
size_t select_lds_bytes(int scored_rows, int descriptor_capacity, int max_selected) {
  return (size_t)((scored_rows + 7) & ~7) * 2 + (size_t)descriptor_capacity * DESC_ARRAYS * 4 +
         (size_t)((max_selected + 63) / 64 + 2) * 4;
}

int launch_score_select(const DecodeArgs& a, hipStream_t s, const DecodeArgs* pending) {
  if (large_selection(a))  // scoring (and the pending update) on every compute unit, then the selection
    return launch_select_large(a, s, pending);
  const int ct = a.st.centroid_dtype, dt = a.kv.dtype;
  const int nscore = std::min(a.st.community_capacity, a.ws.score_blocks * SCORE_BLOCK);
  const size_t lds = select_lds_bytes(nscore, a.ws.descriptor_capacity, a.cfg.max_selected);
  const int own = (nscore + SELECT_THREADS - 1) / SELECT_THREADS;
  auto launch = [&](auto kernel) {
    if (lds > 48 * 1024) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        return limit_error("selection LDS (communities x 2 + descriptors x 28 + selected / 16 bytes) exceeds the device limit");
      }
    }
    DecodeArgs u;
    memset(&u, 0, sizeof(u));
    int extra = 0;
    if (pending != nullptr && pending->cfg.assignment != CKV_ASSIGN_NONE) {
      u = *pending;
      extra = pending->st.retrieval_heads;
    }
    const int parts = (int)std::max<int64_t>(
        1, std::min<int64_t>(PRESELECT_MAX_PARTS, (CKV_DEVICE_CUS - extra) / std::max(1, a.st.retrieval_heads)));
    hipLaunchKernelGGL(kernel, dim3(a.st.retrieval_heads * parts + extra), dim3(SELECT_THREADS), lds, s, a, u,
                       parts);
    return launch_check("select");
  };
  constexpr int OWN_MAX = CKV_MAX_SELECT_ROWS / SELECT_THREADS;
  auto by_own = [&](auto k1, auto k2, auto kmax) {
    return own <= 1 ? launch(k1) : own <= 2 ? launch(k2) : launch(kmax);
  };
  if (ct == CKV_E4M3 && dt == CKV_BF16) {
    if (own > 2 && own <= 4) return launch(select_kernel<CKV_E4M3, CKV_BF16, 4>);
    return by_own(select_kernel<CKV_E4M3, CKV_BF16, 1>, select_kernel<CKV_E4M3, CKV_BF16, 2>,
                  select_kernel<CKV_E4M3, CKV_BF16, OWN_MAX>);
  }
  if (ct == CKV_E4M3)
    return by_own(select_kernel<CKV_E4M3, CKV_F32, 1>, select_kernel<CKV_E4M3, CKV_F32, 2>,
                  select_kernel<CKV_E4M3, CKV_F32, OWN_MAX>);
  if (dt == CKV_BF16)
    return by_own(select_kernel<CKV_F32, CKV_BF16, 1>, select_kernel<CKV_F32, CKV_BF16, 2>,
                  select_kernel<CKV_F32, CKV_BF16, OWN_MAX>);
  return by_own(select_kernel<CKV_F32, CKV_F32, 1>, select_kernel<CKV_F32, CKV_F32, 2>,
                select_kernel<CKV_F32, CKV_F32, OWN_MAX>);
}

// Parts per head of the fused selection + attention path (64-slot tiles of
// the slot table, eight per workgroup), or 0 when the path cannot serve `a`:
// bf16 KV, a materialised slot table of at most 8192 slots held in LDS, and a
// query group small enough for the wide split merge.
int fused_parts(const DecodeArgs& a) {
  if (a.kv.dtype != CKV_BF16 || a.csr.member_offsets == nullptr) return 0;
  if (a.ws.slot_capacity > 8192 || a.cfg.group_size * D > 512) return 0;
  const int tiles = a.ws.slot_capacity / TILE;
  const int parts = (tiles + FUSED_TILES - 1) / FUSED_TILES;
  const size_t lds = fused_lds_bytes(a);
  return (parts <= 64 && lds <= FUSED_LDS_LIMIT) ? parts : 0;
}

size_t fused_lds_bytes(const DecodeArgs& a) {
  const int parts = (a.ws.slot_capacity / TILE + FUSED_TILES - 1) / FUSED_TILES;
  return fused_slot_bytes(a.ws.slot_capacity) + fused_select_bytes(a.st.community_capacity, a.ws.budget_tiles, parts) +
         attend_part_lds_bytes(SELECT_THREADS / 64);
}

// Compute units of the current device (cached per device).
int compute_units() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

int coop_parts(const DecodeArgs& a) {
  const int parts = fused_parts(a);
  if (parts == 0 || parts > COOP_MAX_PARTS || a.ws.exchange == nullptr || a.st.centroid_dtype != CKV_E4M3) return 0;
  // Every part polls for the other parts' scores: the whole grid (with one
  // pending-update workgroup per head) must be resident at once, one
  // workgroup per compute unit; a larger layer takes the separate launches
  // (8 heads x 34 parts at a 4,096-token budget: 293 against 535 us for 8
  // such sequences, the parts that could not start leaving the others
  // polling until they scored every community themselves).
  if ((int64_t)a.st.retrieval_heads * (parts + 1) > compute_units()) return 0;
  return a.st.community_capacity <= 4 * SELECT_THREADS ? parts : 0;
}

int launch_select_attend(const DecodeArgs& a, hipStream_t s, const DecodeArgs* pending, int parts, bool coop) {
  const size_t lds = fused_lds_bytes(a);
  const int nscore = std::min(a.st.community_capacity, a.ws.score_blocks * SCORE_BLOCK);
  const int own = (nscore + SELECT_THREADS - 1) / SELECT_THREADS;
  auto launch = [&](auto kernel) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return limit_error("fused selection + attention LDS exceeds the device limit");
    }
    DecodeArgs u;
    memset(&u, 0, sizeof(u));
    int extra = 0;
    if (pending != nullptr && pending->cfg.assignment != CKV_ASSIGN_NONE) {
      u = *pending;
      extra = pending->st.retrieval_heads;
    }
    hipLaunchKernelGGL(kernel, dim3(a.st.retrieval_heads * parts + extra), dim3(SELECT_THREADS), lds, s, a, u,
                       parts);
    return launch_check("select_attend");
  };
  constexpr int OWN_MAX = CKV_MAX_SELECT_ROWS / SELECT_THREADS;
  if (coop) {
    if (coop_parts(a) != parts) return limit_error("the cooperative fused launch cannot serve this layer");
    // the merge loads PMAX accumulators per output element (clamped to the parts)
    auto by_own = [&](auto k1, auto k2, auto k4) { return own <= 1 ? launch(k1) : own <= 2 ? launch(k2) : launch(k4); };
    if (parts <= 18)
      return by_own(select_attend_kernel<CKV_E4M3, CKV_BF16, 1, 18>, select_attend_kernel<CKV_E4M3, CKV_BF16, 2, 18>,
                    select_attend_kernel<CKV_E4M3, CKV_BF16, 4, 18>);
    if (parts <= 24)
      return by_own(select_attend_kernel<CKV_E4M3, CKV_BF16, 1, 24>, select_attend_kernel<CKV_E4M3, CKV_BF16, 2, 24>,
                    select_attend_kernel<CKV_E4M3, CKV_BF16, 4, 24>);
    if (parts <= 40)
      return by_own(select_attend_kernel<CKV_E4M3, CKV_BF16, 1, 40>, select_attend_kernel<CKV_E4M3, CKV_BF16, 2, 40>,
                    select_attend_kernel<CKV_E4M3, CKV_BF16, 4, 40>);
    return by_own(select_attend_kernel<CKV_E4M3, CKV_BF16, 1, 64>, select_attend_kernel<CKV_E4M3, CKV_BF16, 2, 64>,
                  select_attend_kernel<CKV_E4M3, CKV_BF16, 4, 64>);
  }
  if (a.st.centroid_dtype == CKV_E4M3) {
    return own <= 1 ? launch(select_attend_kernel<CKV_E4M3, CKV_BF16, 1>)
           : own <= 2 ? launch(select_attend_kernel<CKV_E4M3, CKV_BF16, 2>)
           : own <= 4 ? launch(select_attend_kernel<CKV_E4M3, CKV_BF16, 4>)
                      : launch(select_attend_kernel<CKV_E4M3, CKV_BF16, OWN_MAX>);
  }
  return own <= 1 ? launch(select_attend_kernel<CKV_F32, CKV_BF16, 1>)
         : own <= 2 ? launch(select_attend_kernel<CKV_F32, CKV_BF16, 2>)
                    : launch(select_attend_kernel<CKV_F32, CKV_BF16, OWN_MAX>);
}

int launch_batch_select_attend(const DecodeArgs& h, const DecodeArgs* table, int count, int max_nscore,
                               size_t max_lds, int parts, hipStream_t s) {
  const int own = (max_nscore + SELECT_THREADS - 1) / SELECT_THREADS;
  auto launch = [&](auto kernel) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_lds);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return limit_error("batched fused selection + attention LDS exceeds the device limit");
    }
    hipLaunchKernelGGL(kernel, dim3(count * h.st.retrieval_heads * parts), dim3(SELECT_THREADS), max_lds, s, table,
                       h.st.retrieval_heads, parts);
    return launch_check("select_attend_batch");
  };
  constexpr int OWN_MAX = CKV_MAX_SELECT_ROWS / SELECT_THREADS;
  if (h.st.centroid_dtype == CKV_E4M3) {
    return own <= 1 ? launch(select_attend_batch_kernel<CKV_E4M3, CKV_BF16, 1>)
           : own <= 2 ? launch(select_attend_batch_kernel<CKV_E4M3, CKV_BF16, 2>)
           : own <= 4 ? launch(select_attend_batch_kernel<CKV_E4M3, CKV_BF16, 4>)
                      : launch(select_attend_batch_kernel<CKV_E4M3, CKV_BF16, OWN_MAX>);
  }
  return own <= 1 ? launch(select_attend_batch_kernel<CKV_F32, CKV_BF16, 1>)
         : own <= 2 ? launch(select_attend_batch_kernel<CKV_F32, CKV_BF16, 2>)
                    : launch(select_attend_batch_kernel<CKV_F32, CKV_BF16, OWN_MAX>);
}

// Batched selection of `count` items (bf16 KV); `max_nscore`, `max_lds` are the
// maxima over the items.
// With more than PRESCORE_MIN_ROWS scored rows per head (and no nearest-centroid
// search, which the prescoring does not do) the rows are scored first by
// score_rows_batch_kernel on every compute unit; the selection then loads the
// scores.
constexpr int PRESCORE_MIN_ROWS = 2 * SELECT_THREADS;

int launch_batch_select(const DecodeArgs& h, const DecodeArgs* table, int count, int max_nscore, size_t max_lds,
                        hipStream_t s, const DecodeArgs* utable, int ucount, int uheads) {
  const int extra = utable ? ucount * uheads : 0;  // pending-update workgroups
  const int own = (max_nscore + SELECT_THREADS - 1) / SELECT_THREADS;
  const bool pre = max_nscore > PRESCORE_MIN_ROWS && h.cfg.assignment != CKV_ASSIGN_NEAREST;
  if (pre) {
    const dim3 grid((max_nscore + ROWS_PER_PASS - 1) / ROWS_PER_PASS, count * h.st.retrieval_heads);
    if (h.st.centroid_dtype == CKV_E4M3)
      hipLaunchKernelGGL((score_rows_batch_kernel<CKV_E4M3, CKV_BF16>), grid, dim3(SELECT_THREADS), 0, s, table,
                         h.st.retrieval_heads);
    else
      hipLaunchKernelGGL((score_rows_batch_kernel<CKV_F32, CKV_BF16>), grid, dim3(SELECT_THREADS), 0, s, table,
                         h.st.retrieval_heads);
    const int rc = launch_check("score_rows_batch");
    if (rc) return rc;
  }
  auto set_lds = [&](auto kernel) {
    if (max_lds > 48 * 1024) {
      const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)max_lds);
      if (e != hipSuccess) {
        (void)hipGetLastError();
        return limit_error("batched selection LDS exceeds the device limit");
      }
    }
    return 0;
  };
  auto launch = [&](auto kernel) {
    if (const int rc = set_lds(kernel)) return rc;
    const int nsel = count * h.st.retrieval_heads;
    hipLaunchKernelGGL(kernel, dim3(nsel + extra), dim3(SELECT_THREADS), max_lds, s, table, h.st.retrieval_heads,
                       nsel, utable, uheads);
    return launch_check("select_batch");
  };
  // The prescored selection leaves most compute units idle (one workgroup per
  // (item, head)) while its slot resolution is instruction-bound: `parts`
  // workgroups per (item, head) repeat the selection side by side and split
  // the slot blocks, as many as one round of workgroups on the device holds
  // beside the pending-update workgroups.
  const int pre_parts = (int)std::max<int64_t>(
      1, std::min<int64_t>(PRESELECT_MAX_PARTS,
                           std::max<int64_t>(0, (int64_t)CKV_DEVICE_CUS - extra) / ((int64_t)count * h.st.retrieval_heads)));
  auto launch_pre = [&](auto kernel) {
    if (const int rc = set_lds(kernel)) return rc;
    const int nsel = count * h.st.retrieval_heads * pre_parts;
    hipLaunchKernelGGL(kernel, dim3(nsel + extra), dim3(SELECT_THREADS), max_lds, s, table, h.st.retrieval_heads,
                       pre_parts, nsel, utable, uheads);
    return launch_check("select_prescored_batch");
  };
  constexpr int OWN_MAX = CKV_MAX_SELECT_ROWS / SELECT_THREADS;
  if (pre) {
    if (h.st.centroid_dtype == CKV_E4M3) {
      return own <= 4   ? launch_pre(select_prescored_batch_kernel<CKV_E4M3, CKV_BF16, 4>)
             : own <= 8 ? launch_pre(select_prescored_batch_kernel<CKV_E4M3, CKV_BF16, 8>)
                        : launch_pre(select_prescored_batch_kernel<CKV_E4M3, CKV_BF16, OWN_MAX>);
    }
    return own <= 4 ? launch_pre(select_prescored_batch_kernel<CKV_F32, CKV_BF16, 4>)
                    : launch_pre(select_prescored_batch_kernel<CKV_F32, CKV_BF16, OWN_MAX>);
  }
  if (h.st.centroid_dtype == CKV_E4M3) {
    return own <= 1 ? launch(select_batch_kernel<CKV_E4M3, CKV_BF16, 1>)
           : own <= 2 ? launch(select_batch_kernel<CKV_E4M3, CKV_BF16, 2>)
           : own <= 4 ? launch(select_batch_kernel<CKV_E4M3, CKV_BF16, 4>)
                      : launch(select_batch_kernel<CKV_E4M3, CKV_BF16, OWN_MAX>);
  }
  return own <= 1 ? launch(select_batch_kernel<CKV_F32, CKV_BF16, 1>)
         : own <= 2 ? launch(select_batch_kernel<CKV_F32, CKV_BF16, 2>)
                    : launch(select_batch_kernel<CKV_F32, CKV_BF16, OWN_MAX>);
}

}  // namespace ckv

#ifdef CKV_PHASE_TIMING
extern "C" int ckv_phase_stamps_select(unsigned long long* out) {
  return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(ckv::phase_stamp), sizeof(unsigned long long) * 32);
}
#endif
