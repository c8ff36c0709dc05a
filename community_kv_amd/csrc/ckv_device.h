// Device-side building blocks shared by the decode kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "../../include/ckv_amd.h"
#include "ckv_numerics.h"

namespace ckv {

// Phase timestamps (100 MHz wall clock) for latency-profiling builds compiled
// with -DCKV_PHASE_TIMING; each kernel file then defines its own
// copy of the `phase_stamp` array and a host getter.  Expands to nothing otherwise.
#ifdef CKV_PHASE_TIMING
namespace {
__device__ unsigned long long phase_stamp[32];  // one array per kernel file
}  // namespace
#define CKV_STAMP(cond, slot)                                         \
  do {                                                               \
    if ((cond) && threadIdx.x == 0) phase_stamp[(slot)] = wall_clock64(); \
  } while (0)
#define CKV_STAMP_MAX(cond, slot)                                                            \
  do {                                                                                       \
    if ((cond) && threadIdx.x == 0) atomicMax(&phase_stamp[(slot)], (unsigned long long)wall_clock64()); \
  } while (0)
#define CKV_STAMP_AT(cond, slot)                 \
  do {                                           \
    if (cond) phase_stamp[(slot)] = wall_clock64(); \
  } while (0)
// Register-held stamps (no store until the flush, so no memory wait covers them).
#define CKV_TS_DECL unsigned long long ckv_ts[32] = {}
#define CKV_TS_ARG , unsigned long long* ckv_ts
#define CKV_TS_PASS , ckv_ts
#define CKV_TS(slot) (ckv_ts[(slot)] = wall_clock64())
#define CKV_TS_FLUSH(cond)                                                        \
  do {                                                                            \
    if ((cond) && threadIdx.x == 0)                                               \
      for (int i_ = 0; i_ < 32; ++i_) if (ckv_ts[i_]) phase_stamp[i_] = ckv_ts[i_]; \
  } while (0)
#else
#define CKV_TS_DECL do {} while (0)
#define CKV_TS_ARG
#define CKV_TS_PASS
#define CKV_TS(slot) do {} while (0)
#define CKV_TS_FLUSH(cond) do {} while (0)
#define CKV_STAMP(cond, slot) \
  do {                        \
  } while (0)
#define CKV_STAMP_MAX(cond, slot) \
  do {                            \
  } while (0)
#define CKV_STAMP_AT(cond, slot) \
  do {                           \
  } while (0)
#endif

constexpr int D = CKV_HEAD_DIM;
constexpr int TILE = CKV_TILE;
constexpr int KAPPA = CKV_KAPPA;
constexpr int SCORE_BLOCK = CKV_SCORE_BLOCK;
constexpr int SELECT_THREADS = 512;  // one selection workgroup per retrieval head
constexpr int REDUCE_THREADS = 128;
constexpr float NEG_INF = -__builtin_huge_valf();

// Words (uint64) of one retrieval head's row of the fused launch's exchange
// buffer: the epoch-tagged centroid scores (one per community), then the
// tagged nearest-centroid minima (eight waves of at most 64 parts each) and as
// many reserved words.
__host__ __device__ inline int64_t ckv_exchange_words(int community_capacity) {
  return (int64_t)community_capacity + 2 * 64 * 8;
}

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

// Hardware conversions of gfx950 (single instructions).  Each matches the
// library's reference rounding bit for bit (IEEE round-to-nearest-even, OCP
// e4m3); ckv_device_numerics exposes them for the parity tests.
__device__ inline uint16_t f16_bits_hw(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

__device__ inline uint32_t pack_bf16x2_hw(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ inline float e4m3_to_f32_hw(uint32_t code) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = __builtin_amdgcn_cvt_pk_f32_fp8((int)code, false);
  return v[0];
}

// Loads through the global address space (global_load_*, never flat), so that
// waits on LDS traffic do not also wait on these.
// Non-temporal 16-byte load, for the cooperative launch's K/V row gathers
// (rows read once per step): 16.6 against 17.4 us per config-2 layer-step
// with plain loads.  The tile kernel's gathers measured slower with it.
__device__ inline uint4 gload16_nt(const void* p) {
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return uint4{v[0], v[1], v[2], v[3]};
}

__device__ inline uint4 gload16(const void* p) {
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  typedef const __attribute__((address_space(1))) u32x4_t* global_u32x4_ptr;
  const u32x4_t v = *(global_u32x4_ptr)(p);
  return uint4{v[0], v[1], v[2], v[3]};
}

__device__ inline int32_t gload_i32(const int32_t* p) {
  typedef const __attribute__((address_space(1))) int32_t* global_i32_ptr;
  return *(global_i32_ptr)(p);
}

__device__ inline float gload_f32(const float* p) {
  typedef const __attribute__((address_space(1))) float* global_f32_ptr;
  return *(global_f32_ptr)(p);
}

// Loads and stores for data that workgroups of one launch hand to each other.
// Each XCD's L2 caches device memory without coherence with the other XCDs;
// agent-scope relaxed atomics compile to global_load/global_store with sc1,
// which bypass those copies, so a value stored this way (and waited for) is
// seen by such a load on any compute unit.
__device__ inline uint64_t ld_agent_u64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline uint32_t ld_agent_u32(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline float ld_agent_f32(const float* p) {
  return __uint_as_float(ld_agent_u32(reinterpret_cast<const uint32_t*>(p)));
}
__device__ inline void st_agent_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent_u32(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_agent_f32(float* p, float v) {
  st_agent_u32(reinterpret_cast<uint32_t*>(p), __float_as_uint(v));
}
// A store that stays in this XCD's L2 (workgroup scope: L1 is write-through,
// nothing is written through to memory).  Another workgroup on the same XCD
// sees it with ld_agent_* (which bypasses L1 and hits that L2) after about a
// quarter of a microsecond; one on another XCD does not see it before the
// kernel ends, so data handed over this way carries a tag that the reader
// checks, with a fallback when it never shows.
__device__ inline void st_xcd_u64(uint64_t* p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
// Waits until every global load and store this thread issued has completed.
__device__ inline void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }


// ---------------------------------------------------------------------------
// Cross-lane moves on the VALU (DPP and the gfx950 permlane swaps).  A lone
// wave pays the full latency of every dependent instruction, and an LDS
// permute costs several times a DPP move, so reductions and scans use these.
// ---------------------------------------------------------------------------

__device__ inline int lane_id() { return (int)__lane_id(); }

// Orders this wave's LDS accesses (writes before the barrier are visible to
// every lane of the wave after it) without synchronising other waves.
__device__ inline void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int CTRL>
__device__ inline uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}

// Value held by lane (lane ^ X), X in {1, 2, 4, 8, 16, 32}.
template <int X>
__device__ inline uint32_t xor_u32(uint32_t v) {
  if constexpr (X == 1) {
    return dpp_u32<0xB1>(v);  // quad_perm [1,0,3,2]
  } else if constexpr (X == 2) {
    return dpp_u32<0x4E>(v);  // quad_perm [2,3,0,1]
  } else if constexpr (X == 4) {
    return dpp_u32<0x141>(dpp_u32<0x1B>(v));  // half-row mirror of the quad reverse
  } else if constexpr (X == 8) {
    return dpp_u32<0x141>(dpp_u32<0x140>(v));  // half-row mirror of the row mirror
  } else if constexpr (X == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane_id() & 16) ? (uint32_t)r[0] : (uint32_t)r[1];
  } else {
    static_assert(X == 32, "xor distance");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane_id() & 32) ? (uint32_t)r[0] : (uint32_t)r[1];
  }
}

template <int X>
__device__ inline float xor_f32(float v) {
  return ckv_u2f(xor_u32<X>(ckv_f2u(v)));
}

// v + v[lane ^ X] for X in {1, 2, 4}, written so that the compiler folds the
// last lane move into the add (v_add_f32 with a DPP operand): every lane has a
// source under these controls, so the bound-control zero never applies.
template <int X>
__device__ inline float add_xor_f32(float v) {
  uint32_t u = ckv_f2u(v);
  if constexpr (X == 4) u = dpp_u32<0x1B>(u);  // quad reverse, then the half-row mirror below
  constexpr int CTRL = X == 1 ? 0xB1 : (X == 2 ? 0x4E : 0x141);
  static_assert(X == 1 || X == 2 || X == 4, "xor distance");
  return v + ckv_u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)u, CTRL, 0xF, 0xF, true));
}

// v + v[lane ^ 16] (resp. 32) on every lane, as one swap and one add.
__device__ inline float add_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(ckv_f2u(v), ckv_f2u(v), false, false);
  return ckv_u2f((uint32_t)r[0]) + ckv_u2f((uint32_t)r[1]);
}
__device__ inline float add_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(ckv_f2u(v), ckv_f2u(v), false, false);
  return ckv_u2f((uint32_t)r[0]) + ckv_u2f((uint32_t)r[1]);
}

__device__ inline float fmax_exact(float a, float b) { return a > b ? a : b; }

__device__ inline float max_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(ckv_f2u(v), ckv_f2u(v), false, false);
  return fmax_exact(ckv_u2f((uint32_t)r[0]), ckv_u2f((uint32_t)r[1]));
}
__device__ inline float max_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(ckv_f2u(v), ckv_f2u(v), false, false);
  return fmax_exact(ckv_u2f((uint32_t)r[0]), ckv_u2f((uint32_t)r[1]));
}

// Wave-wide max (any pairing gives the same max), result on every lane.
__device__ inline int wave_max_i32(int v) {
  v = max(v, (int)xor_u32<1>((uint32_t)v));
  v = max(v, (int)xor_u32<2>((uint32_t)v));
  v = max(v, (int)xor_u32<4>((uint32_t)v));
  v = max(v, (int)xor_u32<8>((uint32_t)v));
  v = max(v, (int)xor_u32<16>((uint32_t)v));
  return max(v, (int)xor_u32<32>((uint32_t)v));
}

__device__ inline float wave_max(float v) {
  v = fmax_exact(v, ckv_u2f(dpp_u32<0xB1>(ckv_f2u(v))));
  v = fmax_exact(v, ckv_u2f(dpp_u32<0x4E>(ckv_f2u(v))));
  v = fmax_exact(v, ckv_u2f(dpp_u32<0x141>(ckv_f2u(v))));
  v = fmax_exact(v, ckv_u2f(dpp_u32<0x140>(ckv_f2u(v))));
  v = max_xor16(v);
  return max_xor32(v);
}

// Butterfly sum in the fixed order xor 32, 16, 8, 4, 2, 1 (bit-reproducible).
__device__ inline float wave_sum_tree(float v) {
  v = add_xor32(v);
  v = add_xor16(v);
  v = v + xor_f32<8>(v);
  v = add_xor_f32<4>(v);
  v = add_xor_f32<2>(v);
  return add_xor_f32<1>(v);
}

template <int CTRL>
__device__ inline uint64_t dpp_u64(uint64_t v) {
  return ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)(v & 0xffffffffu));
}

template <bool MAX>
__device__ inline uint64_t pick_u64(uint64_t a, uint64_t b) {
  return MAX ? (a > b ? a : b) : (a < b ? a : b);
}

template <bool MAX>
__device__ inline uint64_t wave_reduce_u64(uint64_t v) {
  v = pick_u64<MAX>(v, dpp_u64<0xB1>(v));
  v = pick_u64<MAX>(v, dpp_u64<0x4E>(v));
  v = pick_u64<MAX>(v, dpp_u64<0x141>(v));
  v = pick_u64<MAX>(v, dpp_u64<0x140>(v));
  {
    const uint32_t lo = (uint32_t)(v & 0xffffffffu), hi = (uint32_t)(v >> 32);
    const auto rl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    v = pick_u64<MAX>(((uint64_t)(uint32_t)rh[0] << 32) | (uint32_t)rl[0],
                      ((uint64_t)(uint32_t)rh[1] << 32) | (uint32_t)rl[1]);
  }
  {
    const uint32_t lo = (uint32_t)(v & 0xffffffffu), hi = (uint32_t)(v >> 32);
    const auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    v = pick_u64<MAX>(((uint64_t)(uint32_t)rh[0] << 32) | (uint32_t)rl[0],
                      ((uint64_t)(uint32_t)rh[1] << 32) | (uint32_t)rl[1]);
  }
  return v;
}

__device__ inline uint64_t wave_max_u64(uint64_t v) { return wave_reduce_u64<true>(v); }
// Wave-wide OR of a 64-bit value, result on every lane.
__device__ inline uint64_t wave_or_u64(uint64_t v) {
  v |= dpp_u64<0xB1>(v);
  v |= dpp_u64<0x4E>(v);
  v |= dpp_u64<0x141>(v);
  v |= dpp_u64<0x140>(v);
  {
    const uint32_t lo = (uint32_t)(v & 0xffffffffu), hi = (uint32_t)(v >> 32);
    const auto rl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    v = (((uint64_t)(uint32_t)rh[0] << 32) | (uint32_t)rl[0]) | (((uint64_t)(uint32_t)rh[1] << 32) | (uint32_t)rl[1]);
  }
  {
    const uint32_t lo = (uint32_t)(v & 0xffffffffu), hi = (uint32_t)(v >> 32);
    const auto rl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto rh = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    v = (((uint64_t)(uint32_t)rh[0] << 32) | (uint32_t)rl[0]) | (((uint64_t)(uint32_t)rh[1] << 32) | (uint32_t)rl[1]);
  }
  return v;
}


__device__ inline uint64_t wave_min_u64(uint64_t v) { return wave_reduce_u64<false>(v); }

template <int X>
__device__ inline uint64_t xor_u64(uint64_t v) {
  return ((uint64_t)xor_u32<X>((uint32_t)(v >> 32)) << 32) | xor_u32<X>((uint32_t)(v & 0xffffffffu));
}

// Bitonic sort across the 64 lanes, descending (lane 0 holds the largest key).
template <int K, int J>
__device__ inline uint64_t bitonic_stage(uint64_t v, int lane) {
  const uint64_t other = xor_u64<J>(v);
  const bool ascending_block = (lane & K) == 0;  // blocks of the final descending order alternate
  const bool lower = (lane & J) == 0;
  const bool keep_max = ascending_block == lower;
  // keep_max lanes take the larger key, the others the smaller (equal keys: either)
  v = ((other > v) == keep_max) ? other : v;
  if constexpr (J > 1) {
    return bitonic_stage<K, J / 2>(v, lane);
  } else {
    return v;
  }
}

template <int K>
__device__ inline uint64_t bitonic_phase(uint64_t v, int lane) {
  v = bitonic_stage<K, K / 2>(v, lane);
  if constexpr (K < 64) {
    return bitonic_phase<K * 2>(v, lane);
  } else {
    return v;
  }
}

__device__ inline uint64_t wave_sort_desc_u64(uint64_t v) { return bitonic_phase<2>(v, lane_id()); }

// Inclusive prefix sum over the 64 lanes: shifts within each row of 16, then
// the row broadcasts of lanes 15 and 31.
__device__ inline int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
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

// Exclusive block scan of two ints over the workgroup; also returns totals.
__device__ inline void block_scan2(int a, int b, int& ea, int& eb, int& ta, int& tb, int* scratch) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ia = wave_inclusive_scan(a);
  const int ib = wave_inclusive_scan(b);
  if (lane == 63) {
    scratch[2 * wave] = ia;
    scratch[2 * wave + 1] = ib;
  }
  __syncthreads();
  int ba = 0, bb = 0;
  ta = 0;
  tb = 0;
  const int waves = (int)(blockDim.x >> 6);
  for (int w = 0; w < waves; ++w) {
    const int xa = scratch[2 * w], xb = scratch[2 * w + 1];
    if (w < wave) {
      ba += xa;
      bb += xb;
    }
    ta += xa;
    tb += xb;
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
  const int prefix = wave_inclusive_scan(local);
  const int total = __builtin_amdgcn_readlane(prefix, 63);
  int above = total - prefix;  // weight of bins above this lane's four
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

// find_threshold_bin's rule with the result on every lane of the calling
// wave (every wave of a workgroup may run it on the same histogram, so no
// barrier is needed to share the result).
__device__ inline void wave_find_bin(const int* hist, int target, int& out_bin, int& out_above) {
  const int lane = threadIdx.x & 63;
  const int b0 = 4 * lane;
  const int4 h = *reinterpret_cast<const int4*>(hist + b0);
  const int hs[4] = {h.x, h.y, h.z, h.w};
  const int prefix = wave_inclusive_scan(h.x + h.y + h.z + h.w);
  const int total = __builtin_amdgcn_readlane(prefix, 63);
  int above = total - prefix;
  int bin = -1, bin_above = 0;
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
    out_bin = -1;
    out_above = 0;
    return;
  }
  const int owner = __ffsll((unsigned long long)hit) - 1;
  out_bin = __builtin_amdgcn_readlane(bin, owner);
  out_above = __builtin_amdgcn_readlane(bin_above, owner);
}

// Host-side launchers (one per translation unit), called after validation.
int launch_score_select(const DecodeArgs& a, hipStream_t stream, const DecodeArgs* pending_update = nullptr);
// More than LARGE_MIN_ROWS (1,024) scored rows per head on the separate
// selection launch: score_rows_kernel on every compute unit (with another
// layer's pending update, same dtypes, on extra workgroups), then
// select_large_kernel (ckv_select_large.hip).
bool large_selection(const DecodeArgs& a);
int launch_select_large(const DecodeArgs& a, hipStream_t stream, const DecodeArgs* pending = nullptr);
int launch_batch_select_large(const DecodeArgs& h, const DecodeArgs* table, int count, int max_nscore,
                              size_t max_lds, hipStream_t stream);
size_t select_large_lds_bytes(const DecodeArgs& a);
int launch_sync_shared(const DecodeArgs& a, hipStream_t stream);
int launch_attention(const DecodeArgs& a, hipStream_t stream, bool partials_only);
int launch_update(const DecodeArgs& a, hipStream_t stream);
// Merge of `splits` bf16 partials (group * 128 <= 512, splits <= 64) + online update in one launch.
int launch_merge_update(const DecodeArgs& a, hipStream_t stream, int splits);
size_t select_lds_bytes(int scored_rows, int descriptor_capacity, int max_selected);
int attention_batch_splits(const DecodeArgs& a);  // 0 when the batched attention cannot serve `a`
int fused_parts(const DecodeArgs& a);              // 0 when the fused selection + attention cannot serve `a`
size_t fused_lds_bytes(const DecodeArgs& a);
// coop: the cooperative variant (scoring shared between a head's workgroups,
// the split merge inside the launch); coop_parts(a) must equal `parts`.
int launch_select_attend(const DecodeArgs& a, hipStream_t stream, const DecodeArgs* pending, int parts, bool coop);
int coop_parts(const DecodeArgs& a);  // parts of the cooperative fused launch, 0 when it cannot serve `a`
int launch_batch_select_attend(const DecodeArgs& h, const DecodeArgs* table, int count, int max_nscore,
                               size_t max_lds, int parts, hipStream_t stream);
int launch_merge(const DecodeArgs& a, hipStream_t stream, int splits);
int launch_batch_merge(const DecodeArgs& h, const DecodeArgs* table, int count, int splits, hipStream_t stream);
// `utable` (null: none): a batch of `ucount` items of `uheads` heads whose
// online update is pending; it runs in extra workgroups of the selection launch.
int launch_batch_select(const DecodeArgs& h, const DecodeArgs* table, int count, int max_nscore, size_t max_lds,
                        hipStream_t stream, const DecodeArgs* utable = nullptr, int ucount = 0, int uheads = 0);
int launch_batch_attention(const DecodeArgs& h, const DecodeArgs* table, int count, hipStream_t stream,
                           bool partials_only = false);
int launch_batch_sync_shared(const DecodeArgs& h, const DecodeArgs* table, int count, hipStream_t stream);
int launch_batch_update(const DecodeArgs& h, const DecodeArgs* table, int count, bool any_shared, hipStream_t stream);
// Merge of `splits` partials and the online update in one launch (+ the shared-graph sync).
int launch_batch_merge_update(const DecodeArgs& h, const DecodeArgs* table, int count, int splits, bool any_shared,
                              hipStream_t stream);
int launch_dense(const DecodeArgs& a, int seq_len, int group, hipStream_t stream);
int launch_check(const char* what);

}  // namespace ckv
