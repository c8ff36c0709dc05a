// MFMA attention tile over gathered KV rows (shared by the attention kernels
// and the fused selection + attention kernel).
#pragma once

#include "ckv_device.h"

namespace ckv {

// ---------------------------------------------------------------------------
// MFMA attention (bf16): one wave per 64-slot tile
// ---------------------------------------------------------------------------
//
// QK^T: v_mfma_f32_16x16x32_bf16 with A = 16 gathered K rows (M = slots,
// K = 32 dims per step) and B = Q^T (N = the query group, zero-padded to 16).
// The 64 slots of a tile are four 16-row sub-tiles; sub-tile j row r holds
// tile slot tau(j, r), chosen so that the accumulator layout (lane l: query
// l % 16, rows 4*(l/16)+i) is exactly the A operand of the P.V MFMA (lane l:
// query l % 16, 8 consecutive K-slots 32*s + 8*(l/16) + u).  P.V: A = P (bf16,
// as the reference rounds P before its dot), B = V^T read from an LDS copy of
// the V tile (16 KB, chunk-swizzled so the four lane groups hit disjoint banks).

constexpr int CKV_DENSE_CHUNK_TILES = 8;  // 512 tokens per dense wave
constexpr int V_HALF_ROWS = 32;          // rows of a V tile staged in LDS at a time

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ inline int tau(int j, int r) { return 32 * (j >> 1) + 8 * (r >> 2) + 4 * (j & 1) + (r & 3); }

// LDS index of element (row, dim) of a 64 x 128 bf16 tile with swizzled 16-byte chunks.
__device__ inline int vidx(int row, int dim) {
  const int chunk = (dim >> 3) ^ (((row >> 3) & 3) << 1);
  return row * D + (chunk << 3) + (dim & 7);
}

__device__ inline f32x4_t mfma_bf16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

__device__ inline uint32_t pack_bf16x2(float lo, float hi) { return pack_bf16x2_hw(lo, hi); }

// ds_read_b64_tr_b16: within each group of 16 lanes, lane i receives element
// i % 4 of the 8-byte words addressed by lanes i / 4 + 4k, k = 0..3.
__device__ inline uint2 lds_read_tr16(const uint16_t* p) {
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4_t* lds_s16x4_ptr;
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(const_cast<uint16_t*>(p)));
  return __builtin_bit_cast(uint2, v);
}

struct QOperand {
  uint4 s[4];  // Q^T B-operand chunks for the four 32-dim steps
};

// Computes one tile: scores (scaled, -inf where pos_s < 0), per-query max and
// sum, and accumulates P.V into o (rows g = 4*(lane/16)+i, dims 16*nb + lane%16).
// Returns through the references; `corr` rescales o before accumulation.
struct TileResult {
  float m;      // tile max of query lane%16 (scaled scores)
  float l;      // sum of exp(score - m)
};

// NH: number of 32-token halves (2: a 64-slot tile, 1: one half; positions are
// then local tokens 0..31 of pos_s).
template <int NH>
__device__ inline TileResult mfma_tile(const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int64_t kbase,
                                       int64_t tstride, const int* pos_s, uint16_t* v_s, float* cand_s,
                                       const QOperand qop, float scale, float m_prev, f32x4_t* o) {
  constexpr int NJ = 2 * NH;  // 16-token MFMA row blocks
  const int lane = threadIdx.x & 63;  // lane within the wave (workgroups may hold several waves)
  const int L = lane >> 4;
  const int c16 = lane & 15;
  // Masked slots (position -1) read row 0 and are masked out of the softmax,
  // so every load is unconditional and all of them are in flight together.
  uint4 kreg[NJ][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int p = max(pos_s[tau(j, c16)], 0);
#pragma unroll
    for (int s = 0; s < 4; ++s) kreg[j][s] = gload16(K + kbase + (int64_t)p * tstride + 32 * s + 8 * L);
  }
  uint4 vreg[8 * NH];
#pragma unroll
  for (int i = 0; i < 8 * NH; ++i) {
    const int p = max(pos_s[4 * i + L], 0);
    vreg[i] = gload16(V + kbase + (int64_t)p * tstride + 8 * c16);  // (non-temporal here: slower, 75.7 against 70.7 us per config-4 step)
  }
  f32x4_t sacc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    sacc[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s) sacc[j] = mfma_bf16(kreg[j][s], qop.s[s], sacc[j]);
  }
  float sc[NJ][4];
  float mloc = NEG_INF;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = pos_s[tau(j, 4 * L + i)] >= 0;
      const float v = ok ? sacc[j][i] * scale : NEG_INF;
      sc[j][i] = v;
      mloc = fmax_exact(mloc, v);
    }
  }
  if (cand_s != nullptr && c16 == 0) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) cand_s[tau(j, 4 * L + i)] = sc[j][i];
    }
  }
  mloc = max_xor16(mloc);
  mloc = max_xor32(mloc);
  TileResult res;
  const float m_new = fmax_exact(m_prev, mloc);
  res.m = m_new;
  float lsum = 0.0f;
  uint32_t pk[NJ][2];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = sc[j][i] == NEG_INF ? 0.0f : __expf(sc[j][i] - m_new);
      lsum = lsum + p[i];
    }
    pk[j][0] = pack_bf16x2(p[0], p[1]);
    pk[j][1] = pack_bf16x2(p[2], p[3]);
  }
  lsum = add_xor16(lsum);
  lsum = add_xor32(lsum);
  res.l = lsum;
  // rescale the running accumulator rows (query 4L+i) by exp(m_prev - m_new) of that query
  if (m_prev != NEG_INF) {
    const float corr_mine = __expf(m_prev - m_new);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float c = __shfl(corr_mine, 4 * L + i, 64);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) o[nb][i] = o[nb][i] * c;
    }
  }
  // P.V in 32-slot halves; each half of the V tile goes through the wave's
  // 8 KB LDS buffer (row 4i+L of the tile -> buffer row 4(i mod 8)+L, swizzled).
#pragma unroll
  for (int s = 0; s < NH; ++s) {
    wave_sync();  // previous half fully read
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      *reinterpret_cast<uint4*>(v_s + vidx(4 * i + L, 8 * c16)) = vreg[8 * s + i];
    }
    wave_sync();  // this half (and the candidates) visible to every lane of the wave
    const uint4 aop = {pk[2 * s][0], pk[2 * s][1], pk[2 * s + 1][0], pk[2 * s + 1][1]};
    // B operand (8 tokens x 16 dims per lane group) by two transposing reads:
    // lane (L, c16) addresses token 8L + 4h + c16/4, dims 16nb + 4(c16%4)..+3
    // and receives tokens 8L + 4h .. +3 of dim 16nb + c16.
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      const int dim = 16 * nb + 4 * (c16 & 3);
      const uint2 lo = lds_read_tr16(v_s + vidx(8 * L + (c16 >> 2), dim));
      const uint2 hi = lds_read_tr16(v_s + vidx(8 * L + 4 + (c16 >> 2), dim));
      const uint4 bop = {lo.x, lo.y, hi.x, hi.y};
      o[nb] = mfma_bf16(aop, bop, o[nb]);
    }
  }
  return res;
}


// Fused-path attention of one part of a retrieval head's slot table.  The
// part's TP 64-slot tiles (tile = part * TP + w; `pos` = the KV position of
// lane l's slot in tile w on the waves w < TP, -1 for none) are spread over
// all W waves of the workgroup, QROWS = 16 slots each, so that every wave's
// dependent chain is short: it gathers its 16 K and V rows, computes Q K^T
// with v_mfma_f32_16x16x32_bf16 (four 32-dim steps; A = K rows, B = Q^T, the
// accumulator holds query lane % 16 for slots 4 * (lane / 16) + i), the
// softmax numerators rounded to bf16 (as the reference rounds P before its
// dot), and P.V with v_mfma_f32_16x16x16_bf16 (A = P straight from that
// accumulator layout, B = V^T by one transposing LDS read per 16-dim block).
// The workgroup then combines its W wave partials into split partial `part`
// (max, sum, unnormalised P.V per query) and writes every slot's position and
// query-0 score (the candidates of the online update's top-8).
// AGENT: the split partials are stored with st_agent_f32 (another workgroup
// of the launch merges them).
constexpr int QROWS = 16;  // slots per wave in attend_part

// LDS index of element (row, dim) of a 16 x 128 bf16 block whose 16-byte
// chunks are XOR-swizzled by the row: the transposing reads (four rows of one
// chunk per lane group) and the row writes are both free of bank conflicts.
__device__ inline int vq_idx(int row, int dim) { return row * D + ((((dim >> 3) ^ row) & 15) << 3) + (dim & 7); }

__device__ inline f32x4_t mfma_bf16_k16(uint2 a, uint2 b, f32x4_t c) {
  typedef short s16x4_t __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b), c,
                                                   0, 0, 0);
}

// `lds` (16-byte aligned) holds attend_part_lds_bytes(W) bytes.
constexpr size_t attend_part_lds_bytes(int waves) {
  return (size_t)waves * (QROWS * D * 2 + QROWS * 4 + QROWS * 4 + 2 * CKV_MAX_GROUP * 4);
}

template <int W, int TP, bool AGENT = false>
__device__ inline void attend_part(const DecodeArgs& a, const int rh, const int part, const int parts,
                                   int pos, unsigned char* lds CKV_TS_ARG) {
  static_assert(W * QROWS == TP * TILE, "the part's tiles are spread over all waves, 16 slots each");
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int L = lane >> 4;
  const int c16 = lane & 15;
  const int tiles = a.ws.slot_capacity / TILE;
  const int G = a.cfg.group_size;
  const int64_t kb = (int64_t)a.st.retrieval_to_kv[rh] * a.kv.head_stride;
  const int64_t ts = a.kv.token_stride;
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.kv.key);
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.kv.value);
  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.kv.query);
  uint16_t* v_s = reinterpret_cast<uint16_t*>(lds) + wave * (QROWS * D);
  float* o_s = reinterpret_cast<float*>(v_s);  // this wave's P.V rows after its slots
  int* pos_all = reinterpret_cast<int*>(lds + (size_t)W * QROWS * D * 2);  // [W * 16]: the part's slots
  float* cand_all = reinterpret_cast<float*>(pos_all + W * QROWS);
  float* wm_s = cand_all + W * QROWS;
  float* wl_s = wm_s + W * CKV_MAX_GROUP;
  const bool want_topk = a.cfg.assignment != CKV_ASSIGN_NONE;

  // the tile waves publish their slots' positions (and the slot table)
  if (wave < TP) {
    const int tile = part * TP + wave;
    const bool in_range = tile < tiles;
    const bool valid = in_range && pos >= 0 && pos < a.kv.capacity;
    pos_all[wave * TILE + lane] = valid ? pos : -1;
    if (in_range) a.ws.slot_positions[(int64_t)rh * a.ws.slot_capacity + tile * TILE + lane] = pos;
  }
  const uint4 zero = {0u, 0u, 0u, 0u};
  QOperand qop;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint4 v = gload16(Q + ((int64_t)rh * G + min(c16, G - 1)) * D + 32 * s + 8 * L);
    qop.s[s] = c16 < G ? v : zero;
  }
  __syncthreads();
  CKV_TS(18);
  // ---- this wave's 16 slots: part slots 16 * wave + r ----
  const int* pq = pos_all + QROWS * wave;
  uint4 kreg[4], vreg[4];
  {
    const int prow = max(pq[c16], 0);  // masked slots read row 0 and are masked out of the softmax
#pragma unroll
    for (int s = 0; s < 4; ++s) kreg[s] = gload16_nt(K + kb + (int64_t)prow * ts + 32 * s + 8 * L);
#pragma unroll
    for (int i = 0; i < 4; ++i) vreg[i] = gload16_nt(V + kb + (int64_t)max(pq[4 * i + L], 0) * ts + 8 * c16);
  }
  bool ok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) ok[i] = pq[4 * L + i] >= 0;
  f32x4_t sacc = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < 4; ++s) sacc = mfma_bf16(kreg[s], qop.s[s], sacc);
  const float scale = a.cfg.softmax_scale;
  float sc[4];
  float m = NEG_INF;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sc[i] = ok[i] ? sacc[i] * scale : NEG_INF;
    m = fmax_exact(m, sc[i]);
  }
  if (want_topk && c16 == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) cand_all[QROWS * wave + 4 * L + i] = sc[i];
  }
  m = max_xor16(m);
  m = max_xor32(m);
  // The part's maximum per query, shared before P.V (the barrier overlaps the
  // V rows' loads), so every wave's numerators are on one scale and the
  // combine below is a plain sum.
  if (L == 0 && c16 < G) wm_s[wave * CKV_MAX_GROUP + c16] = m;
  __syncthreads();
  {
    float M = NEG_INF;
#pragma unroll
    for (int x = 0; x < W; ++x) M = fmax_exact(M, wm_s[x * CKV_MAX_GROUP + min(c16, G - 1)]);
    m = c16 < G ? M : m;  // lanes past the group keep their own (unused) rows finite
  }
  float p[4];
  float l = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = sc[i] == NEG_INF ? 0.0f : __expf(sc[i] - m);
    l = l + p[i];
  }
  l = add_xor16(l);
  l = add_xor32(l);
  const uint2 aop = {pack_bf16x2(p[0], p[1]), pack_bf16x2(p[2], p[3])};
  // V rows to LDS (row 4i + L, dims 8 * c16 .. +7), then P.V per 16-dim block
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(v_s + vq_idx(4 * i + L, 8 * c16)) = vreg[i];
  wave_sync();
  f32x4_t o[8];
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    // lane (L, c16) receives V[4L .. 4L+3][16 nb + c16]
    const uint2 bop = lds_read_tr16(v_s + vq_idx(4 * L + (c16 >> 2), 16 * nb + 4 * (c16 & 3)));
    o[nb] = mfma_bf16_k16(aop, bop, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f});
  }
  wave_sync();  // every lane's V reads are done before the P.V rows reuse the buffer
  CKV_TS(19);
  if (L == 0 && c16 < G) wl_s[wave * CKV_MAX_GROUP + c16] = l;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int g = 4 * L + i;
    if (g < G) {
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) o_s[g * D + 16 * nb + c16] = o[nb][i];
    }
  }
  if (want_topk && wave < TP) {
    const int tile = part * TP + wave;
    if (tile < tiles) a.ws.slot_scores[(int64_t)rh * a.ws.slot_capacity + tile * TILE + lane] = cand_all[wave * TILE + lane];
  }
  __syncthreads();
  CKV_TS(20);
  // Combine the W wave partials (one scale: the part's maximum) into this
  // part's split partial, in wave order.  A wave without a valid slot has
  // P.V rows of zeros.  Every LDS read is issued before the first add.
  for (int i = tid; i < G * D; i += 64 * W) {
    const int g = i >> 7;
    const int d = i & (D - 1);
    float ov[W];
#pragma unroll
    for (int w = 0; w < W; ++w)
      ov[w] = reinterpret_cast<const float*>(reinterpret_cast<uint16_t*>(lds) + w * (QROWS * D))[g * D + d];
    float acc = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) acc = acc + ov[w];
    float* dst = a.ws.partial_acc + (((int64_t)rh * G + g) * parts + part) * D + d;
    if constexpr (AGENT) st_agent_f32(dst, acc); else *dst = acc;
  }
  CKV_TS(22);
  if (tid < G) {
    float lsum = 0.0f;
    float M = NEG_INF;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      lsum = lsum + wl_s[w * CKV_MAX_GROUP + tid];
      M = fmax_exact(M, wm_s[w * CKV_MAX_GROUP + tid]);
    }
    float* pm = a.ws.partial_max + ((int64_t)rh * G + tid) * parts + part;
    float* pl = a.ws.partial_sum + ((int64_t)rh * G + tid) * parts + part;
    if constexpr (AGENT) {
      st_agent_f32(pm, M);
      st_agent_f32(pl, lsum);
    } else {
      *pm = M;
      *pl = lsum;
    }
  }
  CKV_TS(21);
}

}  // namespace ckv
