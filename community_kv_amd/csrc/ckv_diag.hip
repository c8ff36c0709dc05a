// Device-side numerics exposed for parity tests: the exact device functions
// and hardware conversions the decode kernels use, evaluated over an array.
#include "ckv_device.h"
#include "ckv_error.h"

namespace ckv {

__global__ __launch_bounds__(256) void device_numerics_kernel(int op, const float* in, void* out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float x = in[i];
  switch (op) {
    case 0: reinterpret_cast<float*>(out)[i] = ckv_expf(x); break;
    case 1: reinterpret_cast<float*>(out)[i] = ckv_logf(x); break;
    case 2: reinterpret_cast<uint16_t*>(out)[i] = f16_bits_hw(x); break;
    case 3: reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)(pack_bf16x2_hw(x, 0.0f) & 0xffffu); break;
    case 4: reinterpret_cast<uint8_t*>(out)[i] = ckv_f32_to_e4m3(x); break;
    case 5: reinterpret_cast<float*>(out)[i] = e4m3_to_f32_hw((uint32_t)x & 0xffu); break;
    default: break;
  }
}

// ---- latency probes (the cost model of the decode step's dependent chain) ----

__global__ void probe_empty_kernel(int* never) {
  extern __shared__ int probe_lds[];
  if (never && threadIdx.x == 0x7fffffff) never[0] = probe_lds[0];
}

// One thread follows `hops` dependent loads through next[] (a random cycle
// written by the caller); out[0] = elapsed wall-clock ticks, out[1] = the
// index reached (keeps the chain live).  AGENT: loads bypass the L1 (the
// score exchange's and the merge's loads), else plain loads.
template <bool AGENT>
__global__ void probe_chase_kernel(const uint32_t* __restrict__ next, int32_t hops, uint64_t* out) {
  if (threadIdx.x != 0) return;
  uint32_t i = 0;
  const long long t0 = wall_clock64();
  for (int h = 0; h < hops; ++h)
    i = AGENT ? ld_agent_u32(next + i) : gload_i32(reinterpret_cast<const int32_t*>(next) + i);
  const long long t1 = wall_clock64();
  out[0] = (uint64_t)(t1 - t0);
  out[1] = i;
}

// One thread, `hops` dependent agent-scope fetch-and-adds on one word (the
// arrival counter's round trip).
__global__ void probe_atomic_kernel(uint32_t* word, int32_t hops, uint64_t* out) {
  if (threadIdx.x != 0) return;
  uint32_t v = 0;
  const long long t0 = wall_clock64();
  for (int h = 0; h < hops; ++h)  // the increment depends on the previous result: one round trip each
    v = __hip_atomic_fetch_add(word, v == 0xffffffffu ? 2u : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const long long t1 = wall_clock64();
  out[0] = (uint64_t)(t1 - t0);
  out[1] = v;
}

// Two workgroups hand a counter back and forth `hops` times through agent-scope
// stores and polled agent-scope loads (a workgroup-to-workgroup hand-off);
// bounded polls, so both always finish.  out[0] = ticks of workgroup 0.
__global__ void probe_handoff_kernel(uint32_t* word, int32_t hops, uint64_t* out) {
  if (threadIdx.x != 0) return;
  const uint32_t me = blockIdx.x;
  const long long t0 = wall_clock64();
  int failed = 0;
  for (int h = 0; h < hops; ++h) {
    const uint32_t want = 2u * (uint32_t)h + me;
    int polls = 0;
    while (ld_agent_u32(word) != want && ++polls < (1 << 16)) {
    }
    if (polls >= (1 << 16)) {  // the other workgroup is not running: give up
      failed = 1;
      break;
    }
    st_agent_u32(word, want + 1u);
  }
  const long long t1 = wall_clock64();
  if (me == 0) {
    out[0] = (uint64_t)(t1 - t0);
    out[1] = (uint64_t)failed;
  }
}

// Each workgroup writes the id of the XCD (accelerator complex die) it runs
// on to xcc[blockIdx.x]: the placement of a grid's workgroups on the dies.
// (The launch's dynamic LDS size occupies the compute units as the decode
// launch does; the kernel does not touch it.)  HW_REG_XCC_ID: hwreg 20, bits 0-15.
__global__ void probe_xcc_kernel(uint32_t* xcc) {
  if (threadIdx.x == 0) xcc[blockIdx.x] = __builtin_amdgcn_s_getreg(20 | (15 << 11));
}

}  // namespace ckv

extern "C" int ckv_device_numerics(int op, const float* in, void* out, int64_t n, void* stream) {
  if (!in || !out || n < 0) return ckv_internal::set_error(CKV_E_INVALID, "null argument");
  if (op < 0 || op > 5) return ckv_internal::set_error(CKV_E_INVALID, "unknown numerics op");
  if (n == 0) return CKV_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(ckv::device_numerics_kernel, dim3((unsigned)blocks), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), op, in, out, n);
  return ckv::launch_check("device_numerics");
}

// Diagnostics, no counterpart in the reference: latency probes behind the
// measured cost model of the decode step.  kind 0: an empty kernel of
// `blocks` x `threads` with `lds_bytes` of dynamic LDS (time a graph of them
// on the host); 1 / 2: `hops` dependent plain / agent-scope loads through the
// uint32 cycle in `buffer` (`bytes` long, written by the caller); 3: `hops`
// dependent agent-scope fetch-and-adds on buffer[0]; 4: `hops` hand-offs
// between two workgroups through buffer[0] (zeroed by the caller); 5: a grid
// of `blocks` x `threads` with `lds_bytes` of dynamic LDS whose workgroup b
// writes the id of the XCD it runs on to ((uint32_t*)buffer)[b].  Kinds 1-4
// write elapsed 100 MHz wall-clock ticks to out[0] (out: 2 uint64, device).
extern "C" int ckv_latency_probe(int32_t kind, void* buffer, int64_t bytes, int32_t hops, int32_t blocks,
                                 int32_t threads, int32_t lds_bytes, uint64_t* out, void* stream) {
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (kind == 0) {
    if (blocks <= 0 || threads <= 0 || threads > 1024 || lds_bytes < 0 || lds_bytes > 160 * 1024)
      return ckv_internal::set_error(CKV_E_INVALID, "bad empty-kernel shape");
    if (lds_bytes > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(ckv::probe_empty_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes) != hipSuccess) {
      (void)hipGetLastError();
      return ckv_internal::set_error(CKV_E_LAUNCH, "dynamic LDS size refused");
    }
    hipLaunchKernelGGL(ckv::probe_empty_kernel, dim3(blocks), dim3(threads), (size_t)lds_bytes, s, nullptr);
    return ckv::launch_check("probe_empty");
  }
  if (!buffer || ((!out || hops <= 0) && kind != 5))
    return ckv_internal::set_error(CKV_E_INVALID, "null probe buffer or no hops");
  uint32_t* b = reinterpret_cast<uint32_t*>(buffer);
  switch (kind) {
    case 1:
    case 2:
      if (bytes < 4) return ckv_internal::set_error(CKV_E_INVALID, "probe buffer too small");
      if (kind == 1) hipLaunchKernelGGL(ckv::probe_chase_kernel<false>, dim3(1), dim3(64), 0, s, b, hops, out);
      else hipLaunchKernelGGL(ckv::probe_chase_kernel<true>, dim3(1), dim3(64), 0, s, b, hops, out);
      break;
    case 3: hipLaunchKernelGGL(ckv::probe_atomic_kernel, dim3(1), dim3(64), 0, s, b, hops, out); break;
    case 4: hipLaunchKernelGGL(ckv::probe_handoff_kernel, dim3(2), dim3(64), 0, s, b, hops, out); break;
    case 5:
      if (blocks <= 0 || threads <= 0 || threads > 1024 || lds_bytes < 0 || lds_bytes > 160 * 1024 ||
          bytes < (int64_t)blocks * 4)
        return ckv_internal::set_error(CKV_E_INVALID, "bad placement-probe shape");
      if (lds_bytes > 64 * 1024 &&
          hipFuncSetAttribute(reinterpret_cast<const void*>(ckv::probe_xcc_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, lds_bytes) != hipSuccess) {
        (void)hipGetLastError();
        return ckv_internal::set_error(CKV_E_LAUNCH, "dynamic LDS size refused");
      }
      hipLaunchKernelGGL(ckv::probe_xcc_kernel, dim3(blocks), dim3(threads), (size_t)lds_bytes, s, b);
      break;
    default: return ckv_internal::set_error(CKV_E_INVALID, "unknown probe kind");
  }
  return ckv::launch_check("latency_probe");
}
