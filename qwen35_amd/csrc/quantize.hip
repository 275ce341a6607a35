// quantize.hip -- activation quantizers, bit-exact with the reference CPU path.
//
//   Q8_0  src/kernels/x86/kernels32.c:1064-1087   per 32 values: f16 scale,
//         q = trunc(x*inv +- 0.5) clamped to [-128, 127]
//   Q8_K  src/kernels/x86/kernels256.c:865-896    per 256 values: f32 scale,
//         q = roundf(x*inv) clamped to [-127, 127] (NaN -> 127), int16 bsums
//
// The library is compiled with -ffp-contract=off: x*inv and the following add
// round separately, exactly as the reference's two statements do, and the
// divisions are IEEE correctly rounded (HIP's default for float '/').
#include "qhip_device.hpp"
#include "qhip_internal.hpp"

namespace qhip {

// One thread per value; 32 consecutive threads form one block (half a wave).
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ x,
                                                        uint8_t* __restrict__ out, long nblocks,
                                                        long x_stride, long out_stride) {
  const long b = ((long)blockIdx.x * 256 + threadIdx.x) >> 5;  // block within the token row
  const int i = threadIdx.x & 31;
  const long t = blockIdx.y;                                  // token
  const bool ok = b < nblocks;
  const float v = ok ? x[t * x_stride + 32 * b + i] : 0.0f;
  uint32_t hb;
  const int q = quant_q8_0_lane(v, hb);
  if (ok) {
    uint8_t* ob = out + t * out_stride + 34 * b;
    ob[2 + i] = (uint8_t)(int8_t)q;
    if (i == 0) {
      ob[0] = (uint8_t)hb;
      ob[1] = (uint8_t)(hb >> 8);
    }
  }
}

// One wave per 256-value block; lane l holds values 4l..4l+3.
__global__ __launch_bounds__(256) void k_quantize_q8_K(const float* __restrict__ x,
                                                        uint8_t* __restrict__ out, long nblocks,
                                                        long x_stride, long out_stride) {
  const long b = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  const long t = blockIdx.y;
  const bool ok = b < nblocks;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = ok ? x[t * x_stride + 256 * b + 4 * l + i] : 0.0f;
  int gsum;
  float scale;
  const uint32_t packed = quant_q8_K_lane(v, gsum, scale);
  if (ok) {
    uint8_t* ob = out + t * out_stride + 292 * b;
    *(uint32_t*)(ob + 4 + 4 * l) = packed;
    if ((l & 3) == 0) *(int16_t*)(ob + 260 + 2 * (l >> 2)) = (int16_t)gsum;
    if (l == 0) *(float*)ob = scale;
  }
}

hipError_t launch_quantize_q8_0(const float* x, void* out, long nblocks, int tokens, long x_stride,
                                long out_stride, hipStream_t s) {
  if (nblocks <= 0 || tokens <= 0) return hipSuccess;
  dim3 grid((unsigned)((nblocks * 32 + 255) / 256), (unsigned)tokens);
  hipLaunchKernelGGL(k_quantize_q8_0, grid, dim3(256), 0, s, x, (uint8_t*)out, nblocks, x_stride,
                     out_stride);
  return hipGetLastError();
}

hipError_t launch_quantize_q8_K(const float* x, void* out, long nblocks, int tokens, long x_stride,
                                long out_stride, hipStream_t s) {
  if (nblocks <= 0 || tokens <= 0) return hipSuccess;
  dim3 grid((unsigned)((nblocks + 3) / 4), (unsigned)tokens);
  hipLaunchKernelGGL(k_quantize_q8_K, grid, dim3(256), 0, s, x, (uint8_t*)out, nblocks, x_stride,
                     out_stride);
  return hipGetLastError();
}

}  // namespace qhip
