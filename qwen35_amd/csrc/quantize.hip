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

typedef float qf32x4 __attribute__((ext_vector_type(4)));

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

// ---- wide forms (16-byte aligned f32 rows) ----------------------------------------
// The blocks are numbered over (token, block) -- g = t nb + b -- so that short
// rows still fill the workgroups, and every lane reads 16-byte pieces.  With a
// packed offset table (ragged) token t is packed token t of its sequence
// (whose rows may be at any 4-byte alignment).
// The arithmetic per value is that of quant_q8_0_lane / quant_q8_K_lane, so
// the bytes are the same.

// The owning sequence of packed token p (off[lo] <= p < off[lo + 1]).
__device__ __forceinline__ int find_seq(const int* __restrict__ off, int nseq, int p) {
  int lo = 0, hi = nseq;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (off[mid] <= p) lo = mid; else hi = mid;
  }
  return lo;
}

// Four floats from p: one 16-byte load, or (CHECK, a row of a ragged batch,
// whose sequence pointers the host cannot see) four 4-byte loads where p is
// not 16-byte aligned.
template <bool CHECK>
__device__ __forceinline__ qf32x4 load4f(const float* p) {
  if (CHECK && ((uintptr_t)p & 15u)) return qf32x4{p[0], p[1], p[2], p[3]};
  return *(const qf32x4*)p;
}

template <bool RAGGED>
__device__ __forceinline__ const float* act_row(const float* x, const float* const* src, const int* off, int nseq,
                                                int t, long x_stride) {
  if constexpr (RAGGED) {
    const int sq = find_seq(off, nseq, t);
    return src[sq] + (long)(t - off[sq]) * x_stride;
  } else {
    return x + (long)t * x_stride;
  }
}

// Q8_0: lane l holds values 8 (l & 3) .. +7 of block l >> 2 (16 blocks per
// wave, 64 per workgroup); the block maximum is a max over the four lanes of
// a quad (DPP).
template <bool RAGGED>
__global__ __launch_bounds__(256) void k_quantize_q8_0w(const float* __restrict__ x, const float* const* __restrict__ src,
                                                         const int* __restrict__ off, int nseq, uint8_t* __restrict__ out,
                                                         int nb, int total, long x_stride, long out_stride) {
  const int g = blockIdx.x * 64 + (threadIdx.x >> 2), pt = threadIdx.x & 3;
  const int gc = g < total ? g : total - 1;
  const int t = gc / nb, b = gc - t * nb;
  const float* xr = act_row<RAGGED>(x, src, off, nseq, t, x_stride) + 32 * b + 8 * pt;
  const qf32x4 v0 = load4f<RAGGED>(xr), v1 = load4f<RAGGED>(xr + 4);
  const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
  // |v| with the reference's "if (a > amax)" NaN handling: NaN never wins
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float e = v[i] < 0.0f ? -v[i] : v[i];
    e = e > 0.0f ? e : 0.0f;
    a = fmaxf(a, e);
  }
  a = fmaxf(a, dpp_f32<0xB1>(a));  // quad_perm [1, 0, 3, 2]
  a = fmaxf(a, dpp_f32<0x4E>(a));  // quad_perm [2, 3, 0, 1]
  const float scale = a > 0.0f ? a / 127.0f : 1.0f;
  const float inv = a > 0.0f ? 1.0f / scale : 0.0f;
  uint32_t w[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float sv = v[i] * inv;
    const float r = sv + (sv >= 0.0f ? 0.5f : -0.5f);
    int q = trunc_i32_x86(r);
    q = q > 127 ? 127 : q;
    q = q < -128 ? -128 : q;
    w[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
  }
  if (g < total) {
    // the block is 2-byte aligned: four 16-bit stores
    uint16_t* ob = (uint16_t*)(out + (long)t * out_stride + 34L * b);
    ob[1 + 4 * pt] = (uint16_t)w[0];
    ob[2 + 4 * pt] = (uint16_t)(w[0] >> 16);
    ob[3 + 4 * pt] = (uint16_t)w[1];
    ob[4 + 4 * pt] = (uint16_t)(w[1] >> 16);
    if (pt == 0) ob[0] = (uint16_t)f32_to_f16_bits(scale);
  }
}

// Q8_K: each wave quantizes four consecutive blocks, their loads issued
// first (lane l holds values 4l..4l+3 of each, as quant_q8_K_lane).
template <bool RAGGED>
__global__ __launch_bounds__(256) void k_quantize_q8_Kw(const float* __restrict__ x, const float* const* __restrict__ src,
                                                         const int* __restrict__ off, int nseq, uint8_t* __restrict__ out,
                                                         int nb, int total, long x_stride, long out_stride) {
  const int g0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 4, l = threadIdx.x & 63;
  qf32x4 v[4];
  int tk[4], bk[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int gc = g0 + k < total ? g0 + k : total - 1;
    tk[k] = gc / nb;
    bk[k] = gc - tk[k] * nb;
    v[k] = load4f<RAGGED>(act_row<RAGGED>(x, src, off, nseq, tk[k], x_stride) + 256L * bk[k] + 4 * l);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (g0 + k >= total) break;  // uniform over the wave
    const float vv[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
    int gsum;
    float scale;
    const uint32_t packed = quant_q8_K_lane(vv, gsum, scale);
    uint8_t* ob = out + (long)tk[k] * out_stride + 292L * bk[k];
    *(uint32_t*)(ob + 4 + 4 * l) = packed;
    if ((l & 3) == 0) *(int16_t*)(ob + 260 + 2 * (l >> 2)) = (int16_t)gsum;
    if (l == 0) *(float*)ob = scale;
  }
}

static bool wide_ok(const float* x, long x_stride) {
  return ((uintptr_t)x & 15u) == 0 && (x_stride & 3) == 0;
}

// Blocks (tokens x blocks per row) from which the wide forms run.  Measured
// on MI355X: Q8_0 [1673, 1024] 3.7 against 6.2 us (ragged 4.0 against 7.3),
// but [512, 1024] 3.7 against 3.5 and one token of 2560 / 5120 values 0.1-0.2
// us slower (a few workgroups); Q8_K [512, 17408] 11.9 against 13.0 us, but
// [512, 5120] 5.9 against 5.7 and the ragged [1673, 5120] 17.5 against 13.4
// (the per-block sequence search), so the ragged Q8_K packer keeps the
// one-block-per-wave form.
constexpr long kWideMinBlocks = 32768;
bool quantize_wide_preferred(long blocks) { return blocks >= kWideMinBlocks; }

hipError_t launch_quantize_wide(bool q8_0, const float* x, const float* const* src, const int* off, int nseq,
                                void* out, long nblocks, int tokens, long x_stride, long out_stride,
                                hipStream_t s) {
  const long total = nblocks * tokens;
  if (total <= 0) return hipSuccess;
  if (total > 0x7FFFFFFFL) return hipErrorInvalidValue;
  const bool rag = src != nullptr;
  if (q8_0) {
    const unsigned grid = (unsigned)((total + 63) / 64);
    if (rag)
      hipLaunchKernelGGL(k_quantize_q8_0w<true>, dim3(grid), dim3(256), 0, s, x, src, off, nseq, (uint8_t*)out,
                         (int)nblocks, (int)total, x_stride, out_stride);
    else
      hipLaunchKernelGGL(k_quantize_q8_0w<false>, dim3(grid), dim3(256), 0, s, x, src, off, nseq, (uint8_t*)out,
                         (int)nblocks, (int)total, x_stride, out_stride);
  } else {
    const unsigned grid = (unsigned)((total + 15) / 16);
    if (rag)
      hipLaunchKernelGGL(k_quantize_q8_Kw<true>, dim3(grid), dim3(256), 0, s, x, src, off, nseq, (uint8_t*)out,
                         (int)nblocks, (int)total, x_stride, out_stride);
    else
      hipLaunchKernelGGL(k_quantize_q8_Kw<false>, dim3(grid), dim3(256), 0, s, x, src, off, nseq, (uint8_t*)out,
                         (int)nblocks, (int)total, x_stride, out_stride);
  }
  return hipGetLastError();
}

hipError_t launch_quantize_q8_0(const float* x, void* out, long nblocks, int tokens, long x_stride,
                                long out_stride, hipStream_t s) {
  if (nblocks <= 0 || tokens <= 0) return hipSuccess;
  if (quantize_wide_preferred(nblocks * tokens) && wide_ok(x, tokens > 1 ? x_stride : 0) &&
      ((uintptr_t)out & 1u) == 0 && (out_stride & 1) == 0)
    return launch_quantize_wide(true, x, nullptr, nullptr, 0, out, nblocks, tokens, x_stride, out_stride, s);
  dim3 grid((unsigned)((nblocks * 32 + 255) / 256), (unsigned)tokens);
  hipLaunchKernelGGL(k_quantize_q8_0, grid, dim3(256), 0, s, x, (uint8_t*)out, nblocks, x_stride,
                     out_stride);
  return hipGetLastError();
}

hipError_t launch_quantize_q8_K(const float* x, void* out, long nblocks, int tokens, long x_stride,
                                long out_stride, hipStream_t s) {
  if (nblocks <= 0 || tokens <= 0) return hipSuccess;
  if (quantize_wide_preferred(nblocks * tokens) && wide_ok(x, tokens > 1 ? x_stride : 0))
    return launch_quantize_wide(false, x, nullptr, nullptr, 0, out, nblocks, tokens, x_stride, out_stride, s);
  dim3 grid((unsigned)((nblocks + 3) / 4), (unsigned)tokens);
  hipLaunchKernelGGL(k_quantize_q8_K, grid, dim3(256), 0, s, x, (uint8_t*)out, nblocks, x_stride,
                     out_stride);
  return hipGetLastError();
}

}  // namespace qhip
