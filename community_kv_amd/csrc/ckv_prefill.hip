// Causal prefill attention with per-row top-kappa edge export (gfx950).
//
// Replaces the patched FlashAttention-3 forward of the reference
// (third_party/flash_attention/community-kv.patch: top-8 outputs 31-120,
// fused selection 250-357, WarpSelect 477-723).  Differences by design: the
// per-row selection is exact (the reference keeps six candidates per lane and
// merges four lanes, an approximation), kappa is a parameter (<= 16) and the
// stored value can be the reference probability or the dequantised raw score.
//
// prefill_mfma_kernel: one workgroup = 8 waves = 256 packed rows
// (row r <-> position r / G, query head kv_head * G + r % G, PackGQA), so every
// K/V tile staged in LDS serves all G query heads of the KV head.  Each wave
// owns 32 packed rows and computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16:
// the accumulator puts one query row in each lane (lane % 32) and 16 of the
// tile's keys per lane half, so the row max / sum / top-kappa are per-lane
// register work plus one lane ^ 32 exchange.  O^T = V^T P^T uses the same row
// mapping; V^T operands come from LDS with ds_read_b64_tr_b16.
//
// Top-kappa: each lane keeps a sorted queue of packed keys
// (quantised score << 17 | column + 1) for the columns of its half.  A tile is
// inspected only when some lane's tile maximum reaches its threshold (a lower
// bound of the row's kappa-th best key); candidates above it are appended to a
// small unsorted per-lane buffer, and a wave merges its buffers into the
// queues (sorting network + bitonic merge) only when one would overflow.  The
// two halves' queues are merged exactly at the end.
#include <hip/hip_runtime.h>

#include <float.h>
#include <stdio.h>
#include <string.h>

#include <type_traits>

#include "ckv_device.h"
#include "ckv_error.h"

namespace {
using namespace ckv;

constexpr int D = CKV_HEAD_DIM;
constexpr int PF_WAVES = 8;
constexpr int PF_ROWS = 32 * PF_WAVES;  // packed (position, head) rows per workgroup
constexpr int PF_KEYS = 64;             // keys per LDS tile
constexpr int K_STRIDE = D + 8;         // 272-byte (17-chunk) K rows: 16-lane b128 reads hit distinct banks
constexpr int V_STRIDE = D + 32;        // 320-byte (20-chunk) V rows: transposed b64 reads hit distinct banks
constexpr int K_TILE = PF_KEYS * K_STRIDE;
constexpr int V_TILE = PF_KEYS * V_STRIDE;
constexpr int STAGE = K_TILE + V_TILE;  // elements per pipeline stage
constexpr int PF_STAGES = 3;
constexpr size_t PF_STAGE_BYTES = PF_STAGES * STAGE * sizeof(uint16_t);
// Per-lane top-kappa queues live in LDS after the stages: entry block j
// (entries 4 j .. 4 j + 3) of thread tid at 16 (j * threads + tid); the
// pending-candidate buffers follow, entry e of thread tid at 4 (e * threads + tid).
constexpr int PF_BUF = 8;
// Columns per candidate group: a group is inspected only when its maximum
// reaches the filter (4 measured faster than 2 or 8).
constexpr int PF_GROUP = 4;
template <int QN>
constexpr size_t pf_lds_bytes() { return PF_STAGE_BYTES + (size_t)(QN + PF_BUF) * 4 * 64 * PF_WAVES; }
constexpr int MAX_KAPPA = 16;
constexpr int MAX_SEQ = (1 << 17) - 1;  // column + 1 must fit the 17-bit index field
constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float RESCALE_LOG2 = 8.0f;
// s_waitcnt immediate for vmcnt(0) (expcnt and lgkmcnt left at their maxima).
constexpr int VMCNT0 = 0x0F70;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ inline f32x16_t mfma32(uint4 a, uint4 b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

__device__ inline uint2 lds_tr16(const uint16_t* p) {
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_ptr;
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(uint2, v);
}

// global_load_lds_dwordx4 with an SGPR base and a per-lane byte offset: lane
// i's 16 bytes land at LDS byte address lds_addr + 16 i.  Written as inline
// assembly so that the compiler does not order this wave's LDS reads behind
// it; the caller waits (vmcnt) and synchronises before reading the chunks.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ inline void lds_dma16(const void* gbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(gbase), "s"(lds_addr)
               : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ inline uint32_t swap32_u32(uint32_t v) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return (lane_id() & 32) ? (uint32_t)r[0] : (uint32_t)r[1];
}

// Reference quantisation (community-kv.patch:508-512), float32 operations:
// clamp(rint((s + 48) * 256), 0, 32767).
__device__ inline uint32_t quantise_score(float s) {
  float k = __fmul_rn(__fadd_rn(s, 48.0f), 256.0f);
  k = __builtin_rintf(k);
  k = __builtin_amdgcn_fmed3f(k, 0.0f, 32767.0f);
  return (uint32_t)k;
}

// Scores below this cannot reach a packed key above `thr`: quantise(s) >= key
// needs rint(fl(s + 48) * 256) >= key, i.e. fl(s + 48) >= (key - 0.5) / 256,
// and fl(s + 48) exceeds s + 48 by at most 2^-18 (below 128), so
// s >= (key - 0.5) / 256 - 48 - 2^-18.  The margin 0.504 / 256 covers that
// and the rounding of this expression.  An empty threshold admits every finite
// score.
__device__ inline float prefilter(uint32_t thr) {
  const uint32_t key = thr >> 17;
  return key == 0 ? -FLT_MAX : __builtin_fmaf((float)key, 1.0f / 256.0f, -(48.0f + 0.504f / 256.0f));
}

// Compare-exchange into descending order.
__device__ inline void ce_desc(uint32_t& a, uint32_t& b) {
  const uint32_t hi = max(a, b), lo = min(a, b);
  a = hi;
  b = lo;
}

// Descending sort of 8 keys: the 19-comparator network (Knuth, TAOCP vol. 3,
// 5.3.4, optimal for n = 8), six rounds.
__device__ inline void sort8_desc(uint32_t (&b)[8]) {
  ce_desc(b[0], b[2]); ce_desc(b[1], b[3]); ce_desc(b[4], b[6]); ce_desc(b[5], b[7]);
  ce_desc(b[0], b[4]); ce_desc(b[1], b[5]); ce_desc(b[2], b[6]); ce_desc(b[3], b[7]);
  ce_desc(b[0], b[1]); ce_desc(b[2], b[3]); ce_desc(b[4], b[5]); ce_desc(b[6], b[7]);
  ce_desc(b[2], b[4]); ce_desc(b[3], b[5]);
  ce_desc(b[1], b[4]); ce_desc(b[3], b[6]);
  ce_desc(b[1], b[2]); ce_desc(b[3], b[4]); ce_desc(b[5], b[6]);
}

template <int QN>
__global__ __launch_bounds__(64 * PF_WAVES, 2) void prefill_mfma_kernel(ckv_prefill_args a, int group, int blocks) {
  extern __shared__ __align__(16) uint16_t pf_lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int row = lane & 31;
  const int half = lane >> 5;
  const int kv_heads = a.kv_heads;
  // Longest (latest) row blocks first; consecutive workgroups cycle over the KV
  // heads, so each XCD streams the K/V of few heads through its L2.
  const int blk = blocks - 1 - (int)(blockIdx.x / kv_heads);
  const int kvh = (int)(blockIdx.x % kv_heads);
  const int S = a.seq_len;
  const int64_t pr0 = (int64_t)blk * PF_ROWS;
  const int64_t pr = pr0 + wave * 32 + row;
  const int pos = (int)(pr / group);
  const int head = kvh * group + (int)(pr % group);
  const bool row_ok = pos < S;
  const int pos_lo = (int)(pr0 / group);
  const int pos_hi = min(S - 1, (int)((pr0 + PF_ROWS - 1) / group));
  const int tiles = pos_hi / PF_KEYS + 1;
  const float sl2 = a.softmax_scale * LOG2E;

  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.query);
  const uint16_t* Kg = reinterpret_cast<const uint16_t*>(a.key) + (int64_t)kvh * a.k_head_stride;
  const uint16_t* Vg = reinterpret_cast<const uint16_t*>(a.value) + (int64_t)kvh * a.k_head_stride;
  const int64_t kstride = a.k_row_stride;

  // Q^T B operand: lane (row, half) holds dims 16c + 8 half .. +7 for c = 0..7.
  uint4 qreg[8];
  {
    const uint16_t* qp = Q + (int64_t)(row_ok ? pos : 0) * a.q_row_stride + (int64_t)head * a.q_head_stride + 8 * half;
#pragma unroll
    for (int c = 0; c < 8; ++c) qreg[c] = row_ok ? gload16(qp + 16 * c) : uint4{0u, 0u, 0u, 0u};
  }

  // Staging: K/V tiles go straight from global memory to LDS
  // (global_load_lds_dwordx4: lane i of a wave instruction fills the 16-byte
  // LDS chunk base + i).  A K tile is 64 rows x 17 chunks (16 data + 1 pad),
  // a V tile 64 rows x 20 chunks; wave w issues the instructions n = w + 8 j.
  // Pad chunks load the row's first chunk (never read).  Byte offsets of each
  // lane's source within a tile are fixed; the tile base is uniform.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  int k_src[3], v_src[3];
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const int p = (wave_u + PF_WAVES * j) * 64 + lane;
    const int kc = p % 17;
    k_src[j] = (int)((int64_t)(p / 17) * kstride * 2) + 16 * (kc == 16 ? 0 : kc);
    const int vc = p % 20;
    v_src[j] = (int)((int64_t)(p / 20) * kstride * 2) + 16 * (vc >= 16 ? 0 : vc);
  }
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)pf_lds;
  auto issue_tile = [&](int t, int stage) {
    const uint32_t k_s = lds_base + (uint32_t)(stage * STAGE * 2);
    const uint32_t v_s = k_s + (uint32_t)(K_TILE * 2);
    const int key0 = t * PF_KEYS;
    const char* kb = reinterpret_cast<const char*>(Kg + (int64_t)key0 * kstride);
    const char* vb = reinterpret_cast<const char*>(Vg + (int64_t)key0 * kstride);
    const bool tail = key0 + PF_KEYS > S;  // rows past the sequence re-read row S - 1
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int n = wave_u + PF_WAVES * j;
      int ko = k_src[j], vo = v_src[j];
      if (tail) {
        const int p = n * 64 + lane;
        const int64_t over_k = (int64_t)max(key0 + p / 17 - (S - 1), 0) * kstride * 2;
        const int64_t over_v = (int64_t)max(key0 + p / 20 - (S - 1), 0) * kstride * 2;
        ko -= (int)over_k;
        vo -= (int)over_v;
      }
      if (n < 17) lds_dma16(kb, (uint32_t)ko, k_s + (uint32_t)(n * 1024));
      if (n < 20) lds_dma16(vb, (uint32_t)vo, v_s + (uint32_t)(n * 1024));
    }
  };

  f32x16_t o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int v = 0; v < 16; ++v) o[db][v] = 0.0f;
  }
  // This lane's queue (QN packed keys, descending) in LDS; only its worst
  // entry stays in a register.
  uint4* q_lds = reinterpret_cast<uint4*>(reinterpret_cast<char*>(pf_lds) + PF_STAGE_BYTES) + tid;
#pragma unroll
  for (int j = 0; j < QN / 4; ++j) q_lds[j * 64 * PF_WAVES] = uint4{0u, 0u, 0u, 0u};
  auto load_queue = [&](uint32_t (&q)[QN]) {
#pragma unroll
    for (int j = 0; j < QN / 4; ++j) {
      const uint4 w = q_lds[j * 64 * PF_WAVES];
      q[4 * j] = w.x;
      q[4 * j + 1] = w.y;
      q[4 * j + 2] = w.z;
      q[4 * j + 3] = w.w;
    }
  };
  // This lane's pending candidates (nbuf of PF_BUF, unsorted), entry e at
  // buf_lds[e * threads].
  uint32_t* buf_lds = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(pf_lds) + PF_STAGE_BYTES +
                                                  (size_t)QN * 4 * 64 * PF_WAVES) + tid;
  int nbuf = 0;
  uint32_t q_min = 0u;
  uint32_t row_thr = 0u;  // a lower bound of the row's QN-th best key (both halves)
  // Candidate filter: prefilter(max(own worst kept key, the other half's,
  // row_thr)).  It changes only when the queues do, so it is recomputed there
  // instead of on every tile.
  float tf = -FLT_MAX;
  float m = NEG_INF;  // reference max of the raw score (scale > 0)
  float l = 0.0f;     // this half's share of the softmax denominator

  const int num_sink = a.num_sink;

  // Merges every lane's pending candidates into its queue (called wave-
  // uniformly): drop sink columns, sort the buffer, keep the best QN of queue
  // and buffer (the
  // larger of q[i] and b[QN-1-i] is bitonic; half-cleaners sort it), then
  // refresh the row threshold, i.e. the QN-th best key of the row over both
  // halves' queues, and the filter.
  auto flush = [&]() __attribute__((always_inline)) {
    uint32_t qk[QN];
    load_queue(qk);
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = buf_lds[i * 64 * PF_WAVES];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = (i < nbuf && (int)(b[i] & 0x1ffffu) > num_sink) ? b[i] : 0u;
    sort8_desc(b);
#pragma unroll
    for (int i = (QN > 8 ? QN - 8 : 0); i < QN; ++i) qk[i] = max(qk[i], b[QN - 1 - i]);
#pragma unroll
    for (int j = QN / 2; j >= 1; j >>= 1) {
#pragma unroll
      for (int i = 0; i < QN; ++i) {
        if ((i & j) == 0) ce_desc(qk[i], qk[i + j]);
      }
    }
#pragma unroll
    for (int j = 0; j < QN / 4; ++j) q_lds[j * 64 * PF_WAVES] = uint4{qk[4 * j], qk[4 * j + 1], qk[4 * j + 2], qk[4 * j + 3]};
    q_min = qk[QN - 1];
    nbuf = 0;
    uint32_t rt = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < QN; ++i) rt = min(rt, max(qk[i], swap32_u32(qk[QN - 1 - i])));
    row_thr = rt;
    tf = prefilter(max(max(q_min, swap32_u32(q_min)), row_thr));
  };

  // S^T (keys x rows) of the tile staged in `stage`: accumulator b holds keys
  // 32 b + 8 (v / 4) + 4 half + v % 4 of the tile.
  auto qk_tile = [&](int stage, f32x16_t (&sacc)[2]) __attribute__((always_inline)) {
    const uint16_t* k_s = pf_lds + stage * STAGE;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint4 kf = *reinterpret_cast<const uint4*>(k_s + (32 * b + row) * K_STRIDE + 8 * half);
      sacc[b] = mfma32(kf, qreg[0], f32x16_t{});
    }
#pragma unroll
    for (int c = 1; c < 8; ++c) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const uint4 kf = *reinterpret_cast<const uint4*>(k_s + (32 * b + row) * K_STRIDE + 16 * c + 8 * half);
        sacc[b] = mfma32(kf, qreg[c], sacc[b]);
      }
    }
  };

  // Software pipeline over three LDS stages, diagonal tile first and then
  // backwards (the nearest keys tend to score highest, which raises the
  // top-kappa threshold early).  Iteration t: tile t's scores are in
  // registers, tile t - 1 is resident in LDS and tile t - 2 is in flight.  The
  // QK^T MFMAs of tile t - 1 are issued next to tile t's softmax, so the
  // matrix cores work while the vector ALUs do.
  issue_tile(tiles - 1, 0);
  if (tiles > 1) issue_tile(tiles - 2, 1);
  __builtin_amdgcn_s_waitcnt(VMCNT0);
  __syncthreads();
  f32x16_t sa[2], sb[2];  // this tile's scores / the next tile's, swapped by the two-tile unroll
  qk_tile(0, sa);

  int stage = 0;
  // One tile: `cur` holds tile t's scores; the next tile's QK^T goes into `nxt`.
  auto tile_step = [&](const int t, f32x16_t (&cur)[2], f32x16_t (&nxt)[2]) __attribute__((always_inline)) {
    const int nstage = stage == 2 ? 0 : stage + 1;
    if (t >= 2) issue_tile(t - 2, nstage == 2 ? 0 : nstage + 1);
    const int c0 = t * PF_KEYS;
    // Causal mask: only tiles holding columns past some row's position.
    if (c0 + PF_KEYS - 1 > pos_lo) {
      asm volatile("");  // keeps the masking a branch (not selects on every tile)
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int col = c0 + 32 * b + 8 * (v >> 2) + 4 * half + (v & 3);
          if (col > pos) cur[b][v] = NEG_INF;
        }
      }
    }
    // The lane's tile maximum (three-input maxima); the group maxima are
    // formed only inside the rare inspection below.
    // (this file is compiled with -fno-honor-nans: no NaN-quieting moves
    // before the maxima of MFMA results, which are finite or -inf)
    auto at = [&](int i) { return cur[i >> 4][i & 15]; };
    auto max3 = [](float x, float y, float z) { return __builtin_fmaxf(__builtin_fmaxf(x, y), z); };
    float m3[11];
#pragma unroll
    for (int i = 0; i < 10; ++i) m3[i] = max3(at(3 * i), at(3 * i + 1), at(3 * i + 2));
    m3[10] = max3(at(30), at(31), m3[9]);
    const float lmax = max3(max3(m3[0], m3[1], m3[2]), max3(m3[3], m3[4], m3[5]),
                            max3(m3[6], m3[7], __builtin_fmaxf(m3[8], m3[10])));

    // Top-kappa candidates of this lane's 32 columns, by groups of PF_GROUP
    // columns: every score above the filter goes to the pending buffer
    // (sinks and keys the queue would not keep are dropped by the merge,
    // which is cheaper than testing each candidate), merged first when this
    // group could overflow it.  Placed before the tile's LDS reads are
    // issued, so the rare branch waits for nothing outstanding.
#ifndef CKV_PF_NO_TOPK
    if (__builtin_amdgcn_ballot_w64(lmax >= tf)) {
      constexpr int GS = PF_GROUP, NG = 32 / GS, GPA = 16 / GS;
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        float gmax = cur[g / GPA][GS * (g % GPA)];
#pragma unroll
        for (int e = 1; e < GS; ++e) gmax = __builtin_fmaxf(gmax, cur[g / GPA][GS * (g % GPA) + e]);
        if (__builtin_amdgcn_ballot_w64(gmax >= tf)) {
          int cnt = 0;
#pragma unroll
          for (int e = 0; e < GS; ++e) cnt += cur[g / GPA][GS * (g % GPA) + e] >= tf ? 1 : 0;
          if (__builtin_amdgcn_ballot_w64(nbuf + cnt > PF_BUF)) flush();
#pragma unroll
          for (int e = 0; e < GS; ++e) {
            const int b = g / GPA;
            const int v = GS * (g % GPA) + e;
            const float sv = cur[b][v];
            const int col = c0 + 32 * b + 8 * (v >> 2) + 4 * half + (v & 3);
            if (sv >= tf) {
              buf_lds[nbuf * (64 * PF_WAVES)] =
                  (quantise_score(sv) << 17) | (uint32_t)(col + 1);
              ++nbuf;
            }
          }
        }
      }
    }
#endif

    // Online softmax in base 2 against a reference max m that moves only when
    // a tile exceeds it by more than 2^RESCALE_LOG2 (p <= 2^RESCALE_LOG2 stays
    // exact in float32 and bf16 range); both halves of a row share m.
    const float tmax = max_xor32(lmax);
    const bool grow = tmax > m + RESCALE_LOG2 / sl2;
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? tmax : m;
      const float alpha = m == NEG_INF ? 0.0f : __builtin_amdgcn_exp2f((m - m_new) * sl2);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    }
    const float mc = m == NEG_INF ? 0.0f : m * sl2;  // rows with no key seen yet get p = 0

    // Next tile's scores on the matrix cores while this tile's exponentials run
    // (on the last tile this reads a stale stage and the result is unused).
    qk_tile(nstage, nxt);
    uint32_t pb[2][8];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int v = 0; v < 16; v += 2) {
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(cur[b][v], sl2, -mc));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(cur[b][v + 1], sl2, -mc));
        l += p0;
        l += p1;
        pb[b][v >> 1] = pack_bf16x2_hw(p0, p1);
      }
    }

    // O^T (dims x rows) += V^T P^T over four 16-key chunks.  Chunk kc pairs
    // P registers 8 (kc % 2) .. +7 of accumulator kc / 2 (keys 16 kc + 4 half +
    // e % 4 + 8 (e / 4)) with V^T rows read transposed for the same keys.
    const uint16_t* v_s = pf_lds + stage * STAGE + K_TILE;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const int b = kc >> 1;
      const int vb = 4 * (kc & 1);
      const uint4 bop = uint4{pb[b][vb], pb[b][vb + 1], pb[b][vb + 2], pb[b][vb + 3]};
      const uint16_t* vrow = v_s + (16 * kc + 4 * half + ((lane & 15) >> 2)) * V_STRIDE + 16 * ((lane >> 4) & 1) +
                             4 * (lane & 3);
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const uint2 lo = lds_tr16(vrow + 32 * db);
        const uint2 hi = lds_tr16(vrow + 8 * V_STRIDE + 32 * db);
        o[db] = mfma32(uint4{lo.x, lo.y, hi.x, hi.y}, bop, o[db]);
      }
    }
    __builtin_amdgcn_s_waitcnt(VMCNT0);
    __syncthreads();
    stage = nstage;
  };
  // Software pipeline over three LDS stages, diagonal tile first and then
  // backwards (the nearest keys tend to score highest, which raises the
  // top-kappa threshold early).  Iteration t: tile t's scores are in
  // registers, tile t - 1 is resident in LDS and tile t - 2 is in flight.  The
  // QK^T MFMAs of tile t - 1 are issued next to tile t's softmax, so the
  // matrix cores work while the vector ALUs do.  Two tiles per loop trip, the
  // score buffers alternating, so no accumulator is copied.
  for (int t = tiles - 1; t >= 0; t -= 2) {
    tile_step(t, sa, sb);
    if (t == 0) break;
    tile_step(t - 1, sb, sa);
  }

  if (__builtin_amdgcn_ballot_w64(nbuf > 0)) flush();
  if (!row_ok) return;
  const float l_tot = add_xor32(l);
  const float inv = 1.0f / l_tot;
  const float lse = (m * sl2 + __builtin_amdgcn_logf(l_tot)) * LN2;
  uint16_t* O = reinterpret_cast<uint16_t*>(a.output) + (int64_t)pos * a.o_row_stride + (int64_t)head * a.o_head_stride;
#pragma unroll
  for (int db = 0; db < 4; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dim = 32 * db + 8 * g + 4 * half;
      const uint2 w = uint2{pack_bf16x2_hw(o[db][4 * g] * inv, o[db][4 * g + 1] * inv),
                            pack_bf16x2_hw(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv)};
      *reinterpret_cast<uint2*>(O + dim) = w;
    }
  }
  if (half == 0) a.lse[(int64_t)head * S + pos] = lse;

  // Exact merge of the two halves' sorted queues: the larger of a[i] and
  // b[QN-1-i] is a bitonic sequence holding the best QN of the union.
  uint32_t c[QN];
  load_queue(c);
  uint32_t other[QN];
#pragma unroll
  for (int i = 0; i < QN; ++i) other[i] = swap32_u32(c[i]);
#pragma unroll
  for (int i = 0; i < QN; ++i) c[i] = max(c[i], other[QN - 1 - i]);
#pragma unroll
  for (int j = QN / 2; j >= 1; j >>= 1) {
#pragma unroll
    for (int i = 0; i < QN; ++i) {
      if ((i & j) == 0) {
        const uint32_t hi = max(c[i], c[i + j]);
        const uint32_t lo = min(c[i], c[i + j]);
        c[i] = hi;
        c[i + j] = lo;
      }
    }
  }
  if (pos < a.topk_skip || !a.topk_scores || !a.topk_indices) return;
  const int kappa = a.kappa;
  const int64_t base = ((int64_t)head * a.topk_rows + (pos - a.topk_skip)) * kappa;
#pragma unroll
  for (int i = 0; i < QN; ++i) {
    if (i < kappa) {
      const float deq = (float)(c[i] >> 17) * (1.0f / 256.0f) - 48.0f;
      if (half == 0) {
        a.topk_scores[base + i] = a.score_kind == 0 ? expf(deq * a.softmax_scale - lse) : deq;
      } else {
        a.topk_indices[base + i] = c[i] == 0u ? -1 : (int32_t)(c[i] & 0x1ffffu) - 1;
      }
    }
  }
}

template <int QN>
int launch_prefill(const ckv_prefill_args& a, hipStream_t s) {
  const int group = a.query_heads / a.kv_heads;
  const int64_t packed = (int64_t)a.seq_len * group;
  const int blocks = (int)((packed + PF_ROWS - 1) / PF_ROWS);
  auto kernel = prefill_mfma_kernel<QN>;
  static bool attr_set = false;
  if (!attr_set) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)pf_lds_bytes<QN>());
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return ckv_internal::set_error(CKV_E_LAUNCH, hipGetErrorString(e));
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(kernel, dim3((unsigned)blocks * a.kv_heads), dim3(64 * PF_WAVES), pf_lds_bytes<QN>(), s, a, group,
                     blocks);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ckv_internal::set_error(CKV_E_LAUNCH, hipGetErrorString(e));
  return CKV_OK;
}

}  // namespace

extern "C" int ckv_prefill_attention_topk(const ckv_prefill_args* a, void* stream) {
  if (!a || !a->query || !a->key || !a->value || !a->output || !a->lse) {
    return ckv_internal::set_error(CKV_E_INVALID, "null prefill argument");
  }
  if (a->seq_len <= 0 || a->seq_len > MAX_SEQ) {
    return ckv_internal::set_error(CKV_E_LIMIT, "seq_len must be in [1, 131071] (column + 1 fills a 17-bit field)");
  }
  if (a->kv_heads <= 0 || a->query_heads <= 0 || a->query_heads % a->kv_heads || a->kappa < 1 ||
      a->kappa > MAX_KAPPA) {
    return ckv_internal::set_error(CKV_E_INVALID, "bad head counts or kappa (1..16)");
  }
  if (a->num_sink < 0 || a->topk_skip != a->num_sink + a->kappa - 1 ||
      a->topk_rows != (a->seq_len > a->topk_skip ? a->seq_len - a->topk_skip : 0)) {
    return ckv_internal::set_error(CKV_E_INVALID,
                                   "topk_skip must be num_sink + kappa - 1 and topk_rows seq_len - topk_skip");
  }
  if (a->topk_rows > 0 && (!a->topk_scores || !a->topk_indices)) {
    return ckv_internal::set_error(CKV_E_INVALID, "null top-k output");
  }
  if (!(a->softmax_scale > 0.0f) || (a->score_kind != 0 && a->score_kind != 1)) {
    return ckv_internal::set_error(CKV_E_INVALID, "softmax_scale must be positive and score_kind 0 or 1");
  }
  if (a->q_row_stride % 8 || a->q_head_stride % 8 || a->k_row_stride % 8 || a->k_head_stride % 8 ||
      a->o_row_stride % 4 || a->o_head_stride % 4) {
    return ckv_internal::set_error(CKV_E_INVALID, "q/k/v strides must be multiples of 8 elements, output of 4");
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (a->kappa <= 4) return launch_prefill<4>(*a, s);
  if (a->kappa <= 8) return launch_prefill<8>(*a, s);
  return launch_prefill<16>(*a, s);
}
