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
