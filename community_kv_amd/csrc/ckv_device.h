// Device-side building blocks shared by the decode kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/ckv_amd.h"
#include "ckv_numerics.h"

namespace ckv {


constexpr int D = CKV_HEAD_DIM;
constexpr int TILE = CKV_TILE;
constexpr int KAPPA = CKV_KAPPA;
constexpr int SCORE_BLOCK = CKV_SCORE_BLOCK;
constexpr int SELECT_THREADS = 256;
constexpr int REDUCE_THREADS = 128;
constexpr float NEG_INF = -__builtin_huge_valf();

// Every decode kernel receives the full argument set by value.
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

// Host-side launchers (one per translation unit), called after validation.
int launch_score_select(const DecodeArgs& a, hipStream_t stream);
int launch_attention(const DecodeArgs& a, hipStream_t stream, bool partials_only);
int launch_dense(const DecodeArgs& a, int seq_len, int group, hipStream_t stream);
int launch_check(const char* what);

}  // namespace ckv
