// Centroid scoring arithmetic shared by every scoring path (the selection
// kernels and the cooperative decode launch in ckv_select.hip, the
// prescoring kernels in ckv_select.hip and ckv_select_large.hip): the row
// fragments one lane holds and the pinned-order dot products, so that every
// path produces the same fp16 score bits.
//
// Reference: attention/kernels/centroid_selection.py:32-108 (the scores these
// restate: fp16 of the group maximum of q . bf16(centroid)).
#ifndef CKV_SCORE_H
#define CKV_SCORE_H

#include "ckv_device.h"

namespace ckv {

// Centroid row fragment of one lane: 16 dims (e4m3: 16 bytes, f32: 64 bytes).
template <int CT>
struct CentroidFrag {
  static constexpr int N = CT == CKV_E4M3 ? 1 : 4;
  uint4 v[N];
};

template <int CT>
__device__ inline void load_frag(const void* base, int64_t row, int d0, CentroidFrag<CT>& f) {
  if constexpr (CT == CKV_E4M3) {
    f.v[0] = gload16(reinterpret_cast<const uint8_t*>(base) + row * D + d0);
  } else {
    const float* p = reinterpret_cast<const float*>(base) + row * D + d0;
#pragma unroll
    for (int i = 0; i < 4; ++i) f.v[i] = gload16(p + 4 * i);
  }
}

template <int CT>
__device__ inline void decode_frag(const CentroidFrag<CT>& f, float* out) {
  if constexpr (CT == CKV_E4M3) {
    // Hardware OCP e4m3 -> f32 (exact: every e4m3 value is an f32), two bytes per instruction.
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const uint32_t w[4] = {f.v[0].x, f.v[0].y, f.v[0].z, f.v[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x2_t lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
      const f32x2_t hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
      out[4 * i] = lo[0];
      out[4 * i + 1] = lo[1];
      out[4 * i + 2] = hi[0];
      out[4 * i + 3] = hi[1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[4 * i] = ckv_u2f(f.v[i].x);
      out[4 * i + 1] = ckv_u2f(f.v[i].y);
      out[4 * i + 2] = ckv_u2f(f.v[i].z);
      out[4 * i + 3] = ckv_u2f(f.v[i].w);
    }
  }
}

// One 8-lane group's share of a centroid row's dots with two queries, in the
// pinned order: each lane sums its 16 dims in order (bf16 x e4m3 products have
// at most 12 significant bits, so they are exact in f32 and a fused
// multiply-add equals the pinned multiply-then-add), then the butterfly xor 4,
// 2, 1 adds the lanes.  Shared by the selection's scoring and the prescoring
// kernel so that both give the same bits.
template <int CT, int DT>
__device__ __forceinline__ void dot16_pair(const float* qa, const float* qb, const float* cv, float& a0, float& a1) {
  a0 = qa[0] * cv[0];
  a1 = qb[0] * cv[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    if constexpr (CT == CKV_E4M3 && DT == CKV_BF16) {
      a0 = __builtin_fmaf(qa[i], cv[i], a0);
      a1 = __builtin_fmaf(qb[i], cv[i], a1);
    } else {
      a0 = a0 + qa[i] * cv[i];
      a1 = a1 + qb[i] * cv[i];
    }
  }
  a0 = add_xor_f32<4>(a0);
  a1 = add_xor_f32<4>(a1);
  a0 = add_xor_f32<2>(a0);
  a1 = add_xor_f32<2>(a1);
  a0 = add_xor_f32<1>(a0);
  a1 = add_xor_f32<1>(a1);
}

// Query slice (dims 16*lane8 .. +15) of queries g and g+1 from the LDS copy.
__device__ __forceinline__ void load_q_pair(const float* q_s, int g, int lane8, float* qa, float* qb) {
  const float4* pa = reinterpret_cast<const float4*>(q_s + g * D + 16 * lane8);
  const float4* pq = reinterpret_cast<const float4*>(q_s + (g + 1) * D + 16 * lane8);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float4 x = pa[i], y = pq[i];
    qa[4 * i] = x.x; qa[4 * i + 1] = x.y; qa[4 * i + 2] = x.z; qa[4 * i + 3] = x.w;
    qb[4 * i] = y.x; qb[4 * i + 1] = y.y; qb[4 * i + 2] = y.z; qb[4 * i + 3] = y.w;
  }
}

}  // namespace ckv

#endif  // CKV_SCORE_H
