// Causal prefill attention with per-row top-kappa edge export (gfx950).
//
// Replaces the patched FlashAttention-3 forward of the reference
// (third_party/flash_attention/community-kv.patch: top-8 outputs 31-120,
// fused selection 250-357, WarpSelect 477-723).  Differences by design: the
// per-row selection is exact (the reference keeps six candidates per lane and
// merges four lanes, an approximation), kappa is a parameter (<= 16) and the
// stored value can be the reference probability or the raw q.k score.
//
// prefill_rowwise_kernel: grid (ceil(S/64), query_heads) x 64.  One lane owns
// one query row: q and the output accumulator live in registers, K/V tiles of
// 64 rows are staged through LDS as bf16, the softmax is online per tile, and
// the row's candidates are kept in a sorted register queue of packed
// (quantised score << 17 | column) keys.
#include <hip/hip_runtime.h>

#include <stdio.h>
#include <string.h>

#include "../../include/ckv_amd.h"
#include "ckv_error.h"
#include "ckv_numerics.h"

namespace {

constexpr int D = CKV_HEAD_DIM;
constexpr int ROWS = 64;
constexpr int COLS = 64;
constexpr int MAX_KAPPA = 16;
constexpr float NEG_INF = -__builtin_huge_valf();

// Reference quantisation (community-kv.patch:508-516): key = clamp(rint((s + 48) * 256), 0, 32767).
__device__ inline uint32_t quantise_score(float s) {
  float k = (s + 48.0f) * 256.0f;
  k = __builtin_rintf(k);
  k = k < 0.0f ? 0.0f : (k > 32767.0f ? 32767.0f : k);
  return (uint32_t)k;
}

__global__ __launch_bounds__(ROWS) void prefill_rowwise_kernel(ckv_prefill_args a) {
  const int lane = threadIdx.x;
  const int qh = blockIdx.y;
  const int row0 = blockIdx.x * ROWS;
  const int row = row0 + lane;
  const int S = a.seq_len;
  const int group = a.query_heads / a.kv_heads;
  const int kvh = qh / group;
  const int kappa = a.kappa;
  const float scale = a.softmax_scale;
  const uint16_t* Q = reinterpret_cast<const uint16_t*>(a.query);
  const uint16_t* K = reinterpret_cast<const uint16_t*>(a.key);
  const uint16_t* V = reinterpret_cast<const uint16_t*>(a.value);

  __shared__ uint16_t k_s[COLS][D + 8];
  __shared__ uint16_t v_s[COLS][D + 8];

  const bool row_ok = row < S;
  float q[D];
  float acc[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    q[d] = row_ok ? ckv_bf16_to_f32(Q[(int64_t)row * a.q_row_stride + (int64_t)qh * a.q_head_stride + d]) : 0.0f;
    acc[d] = 0.0f;
  }
  uint32_t qkey[MAX_KAPPA];
  float qraw[MAX_KAPPA];
#pragma unroll
  for (int i = 0; i < MAX_KAPPA; ++i) {
    qkey[i] = 0u;
    qraw[i] = NEG_INF;
  }
  float m = NEG_INF;
  float l = 0.0f;
  const int last_row = min(row0 + ROWS, S) - 1;
  for (int c0 = 0; c0 <= last_row; c0 += COLS) {
    __syncthreads();
    for (int i = lane; i < COLS * (D / 8); i += ROWS) {
      const int r = i / (D / 8);
      const int d8 = (i % (D / 8)) * 8;
      const int c = c0 + r;
      uint4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
      if (c < S) {
        const int64_t off = (int64_t)c * a.k_row_stride + (int64_t)kvh * a.k_head_stride + d8;
        kv = *reinterpret_cast<const uint4*>(K + off);
        vv = *reinterpret_cast<const uint4*>(V + off);
      }
      const uint16_t kw[8] = {(uint16_t)kv.x, (uint16_t)(kv.x >> 16), (uint16_t)kv.y, (uint16_t)(kv.y >> 16),
                              (uint16_t)kv.z, (uint16_t)(kv.z >> 16), (uint16_t)kv.w, (uint16_t)(kv.w >> 16)};
      const uint16_t vw[8] = {(uint16_t)vv.x, (uint16_t)(vv.x >> 16), (uint16_t)vv.y, (uint16_t)(vv.y >> 16),
                              (uint16_t)vv.z, (uint16_t)(vv.z >> 16), (uint16_t)vv.w, (uint16_t)(vv.w >> 16)};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        k_s[r][d8 + e] = kw[e];
        v_s[r][d8 + e] = vw[e];
      }
    }
    __syncthreads();
    if (!row_ok) continue;
    float s[COLS];
    float tile_max = NEG_INF;
    for (int j = 0; j < COLS; ++j) {
      const int c = c0 + j;
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) dot = dot + q[d] * ckv_bf16_to_f32(k_s[j][d]);
      const bool ok = c <= row && c < S;
      s[j] = ok ? dot : NEG_INF;
      if (ok) {
        const float sc = dot * scale;
        tile_max = sc > tile_max ? sc : tile_max;
        if (c >= a.num_sink) {
          const uint32_t cand = (quantise_score(dot) << 17) | ((uint32_t)c & 0x1ffffu);
          if (cand > qkey[kappa - 1]) {
            uint32_t ck = cand;
            float cr = dot;
#pragma unroll
            for (int i = 0; i < MAX_KAPPA; ++i) {
              if (i < kappa && ck > qkey[i]) {
                const uint32_t tk = qkey[i];
                const float tr = qraw[i];
                qkey[i] = ck;
                qraw[i] = cr;
                ck = tk;
                cr = tr;
              }
            }
          }
        }
      }
    }
    if (tile_max == NEG_INF) continue;
    const float m_new = m > tile_max ? m : tile_max;
    const float corr = (m == NEG_INF) ? 0.0f : __expf(m - m_new);
    l = l * corr;
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = acc[d] * corr;
    for (int j = 0; j < COLS; ++j) {
      if (s[j] == NEG_INF) continue;
      const float p = __expf(s[j] * scale - m_new);
      l = l + p;
      const float pb = ckv_bf16_to_f32(ckv_f32_to_bf16_bits(p));
#pragma unroll
      for (int d = 0; d < D; ++d) acc[d] = acc[d] + pb * ckv_bf16_to_f32(v_s[j][d]);
    }
    m = m_new;
  }
  if (!row_ok) return;
  uint16_t* O = reinterpret_cast<uint16_t*>(a.output);
  const float inv = 1.0f / l;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    O[(int64_t)row * a.o_row_stride + (int64_t)qh * a.o_head_stride + d] = ckv_f32_to_bf16_bits(acc[d] * inv);
  }
  const float lse = m + __logf(l);
  a.lse[(int64_t)qh * S + row] = lse;
  if (row >= a.topk_skip && a.topk_scores && a.topk_indices) {
    const int64_t base = ((int64_t)qh * a.topk_rows + (row - a.topk_skip)) * kappa;
    for (int i = 0; i < MAX_KAPPA; ++i) {
      if (i >= kappa) break;
      const uint32_t key = qkey[i] >> 17;
      a.topk_indices[base + i] = (int32_t)(qkey[i] & 0x1ffffu);
      a.topk_scores[base + i] =
          a.score_kind == 0 ? __expf(((float)key * (1.0f / 256.0f) - 48.0f) * scale - lse) : qraw[i];
    }
  }
}

}  // namespace

extern "C" int ckv_prefill_attention_topk(const ckv_prefill_args* a, void* stream) {
  if (!a || !a->query || !a->key || !a->value || !a->output || !a->lse) {
    return ckv_internal::set_error(CKV_E_INVALID, "null prefill argument");
  }
  if (a->seq_len <= 0 || a->seq_len > (1 << 17)) {
    return ckv_internal::set_error(CKV_E_LIMIT, "seq_len must be in [1, 131072] (17-bit column keys)");
  }
  if (a->kv_heads <= 0 || a->query_heads % a->kv_heads || a->kappa < 1 || a->kappa > MAX_KAPPA) {
    return ckv_internal::set_error(CKV_E_INVALID, "bad head counts or kappa (1..16)");
  }
  if (a->topk_skip < 0 || a->topk_rows != (a->seq_len > a->topk_skip ? a->seq_len - a->topk_skip : 0)) {
    return ckv_internal::set_error(CKV_E_INVALID, "topk_rows must equal seq_len - topk_skip");
  }
  if (a->q_row_stride % 8 || a->q_head_stride % 8 || a->k_row_stride % 8 || a->k_head_stride % 8) {
    return ckv_internal::set_error(CKV_E_INVALID, "q/k/v strides must be multiples of 8 elements");
  }
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(prefill_rowwise_kernel, dim3((a->seq_len + ROWS - 1) / ROWS, a->query_heads), dim3(ROWS), 0,
                     s, *a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return ckv_internal::set_error(CKV_E_LAUNCH, hipGetErrorString(e));
  return CKV_OK;
}
