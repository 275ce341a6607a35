// dequant.hip -- GGUF blocks to f32, bit-exact with the reference's dequant
// (src/quant_dequant.zig, the CPU backend's dequantRowInto,
// src/backend_cpu.zig:661-679), for the embedding lookup (Exec.dequantRow,
// src/backend.zig:148-151) and whole-tensor expansion (api.h:95-102).
//
//   Q8_0    d * q                                    quant_dequant.zig:1388-1402
//   IQ4_NL  d * codebook[nibble]                     :347-360
//   Q4_K    (d * sc) * nibble - (dmin * m)           :54-77  (separate roundings)
//   Q6_K    (d * sc) * (q6 - 32)                     :222-251
//   Q5_K    (d * sc) * (nibble + 16 * bit) - (dmin * m)  :188-220
//   Q3_K    (d * (sc - 32)) * q3                      :252-322
//   Q2_K    (d * (sc & 15)) * q2 - (dmin * (sc >> 4)) :892-919
//   IQ4_XS  (d * (ls - 32)) * codebook[nibble]        :324-345
//   Q4_0    (nibble - 8) * d                          :78-88
//   Q4_1    nibble * d + m                            :90-103
//   IQ3_XXS (d * (0.5 + ls) * 0.5) * grid * sign      :417-445
//   IQ3_S   (d * (1 + 2 ls)) * grid * sign            :362-415
// The library is compiled with -ffp-contract=off, so each product and the
// Q4_K difference round exactly as the reference's Zig (strict float mode).
//
// One thread per four consecutive values; the block header is re-read by the
// threads of a block (it is in L1), the quantized bytes once.
#include "qhip_device.hpp"
#include "qhip_internal.hpp"

namespace qhip {

__device__ __forceinline__ uint32_t ld16b(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

__device__ __forceinline__ int iq4_value(uint32_t nib) {
  const uint32_t tab = nib < 4 ? IQ4_T0 : nib < 8 ? IQ4_T1 : nib < 12 ? IQ4_T2 : IQ4_T3;
  return sext8(tab >> (8 * (nib & 3)));
}

template <int TT>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ src, float* __restrict__ dst,
                                                  long nvals) {
  const long v0 = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
  if (v0 >= nvals) return;
  float o[4];
  if constexpr (act32(TT)) {
    constexpr int BB = blk32_bytes(TT);
    const uint8_t* blk = src + (v0 / 32) * BB;
    const int j0 = (int)(v0 % 32);
    const float d = h2f(ld16b(blk));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = j0 + i;
      if constexpr (TT == TT_Q8_0) {
        o[i] = d * (float)(int)(int8_t)blk[2 + j];
      } else if constexpr (TT == TT_IQ4_NL) {
        o[i] = d * (float)iq4_value(j < 16 ? (blk[2 + j] & 15u) : (uint32_t)(blk[2 + j - 16] >> 4));
      } else {  // Q4_0: (q - 8) * d; Q4_1: q * d + m (quant_dequant.zig:78-103)
        constexpr int QO = TT == TT_Q4_1 ? 4 : 2;
        const uint32_t q = j < 16 ? (blk[QO + j] & 15u) : (uint32_t)(blk[QO + j - 16] >> 4);
        if constexpr (TT == TT_Q4_0) o[i] = ((float)q - 8.0f) * d;
        else o[i] = (float)q * d + h2f(ld16b(blk + 2));
      }
    }
  } else if constexpr (TT == TT_Q4_K) {
    const uint8_t* blk = src + (v0 / 256) * 144;
    const int e0 = (int)(v0 % 256), sub = e0 / 32;
    const uint8_t* s12 = blk + 4;
    int sc, m;  // src/kernels/x86/kernels256.c:105-125
    if (sub < 4) {
      sc = s12[sub] & 63;
      m = s12[sub + 4] & 63;
    } else {
      sc = (s12[sub + 4] & 15) | ((s12[sub - 4] >> 6) << 4);
      m = (s12[sub + 4] >> 4) | ((s12[sub] >> 6) << 4);
    }
    const float d1 = h2f(ld16b(blk)) * (float)sc;
    const float m1 = h2f(ld16b(blk + 2)) * (float)m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int l = (e0 + i) % 32;
      const uint32_t q = blk[16 + 32 * (sub / 2) + l];
      const int nib = (int)((sub & 1) ? (q >> 4) : (q & 15u));
      o[i] = d1 * (float)nib - m1;
    }
  } else if constexpr (TT == TT_Q5_K) {  // quant_dequant.zig:188-220
    const uint8_t* blk = src + (v0 / 256) * 176;
    const int e0 = (int)(v0 % 256), sub = e0 / 32;
    const uint8_t* s12 = blk + 4;
    int sc, m;
    if (sub < 4) {
      sc = s12[sub] & 63;
      m = s12[sub + 4] & 63;
    } else {
      sc = (s12[sub + 4] & 15) | ((s12[sub - 4] >> 6) << 4);
      m = (s12[sub + 4] >> 4) | ((s12[sub] >> 6) << 4);
    }
    const float d1 = h2f(ld16b(blk)) * (float)sc;
    const float m1 = h2f(ld16b(blk + 2)) * (float)m;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int l = (e0 + i) % 32;
      const uint32_t q = blk[48 + 32 * (sub / 2) + l];
      const int v = (int)((sub & 1) ? (q >> 4) : (q & 15u)) | (int)(((blk[16 + l] >> sub) & 1u) << 4);
      o[i] = d1 * (float)v - m1;
    }
  } else if constexpr (TT == TT_Q3_K) {  // quant_dequant.zig:252-322
    const uint8_t* blk = src + (v0 / 256) * 110;
    const int e0 = (int)(v0 % 256), g = e0 / 16, c = g / 4;
    const uint32_t a0 = ld16b(blk + 96) | (ld16b(blk + 98) << 16), a1 = ld16b(blk + 100) | (ld16b(blk + 102) << 16);
    const uint32_t a2 = ld16b(blk + 104) | (ld16b(blk + 106) << 16);
    const uint32_t base = (c & 1) ? a1 : a0;
    const uint32_t scw = ((c >= 2 ? (base >> 4) : base) & 0x0F0F0F0Fu) | (((a2 >> (2 * c)) & 0x03030303u) << 4);
    const float dl = h2f(ld16b(blk + 108)) * (float)((int)((scw >> (8 * (g % 4))) & 0xFFu) - 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + i, h = e / 128, j = (e % 128) / 32, l = e % 32;
      const int v = (int)((blk[32 + 32 * h + l] >> (2 * j)) & 3u) - (((blk[l] >> (4 * h + j)) & 1u) ? 0 : 4);
      o[i] = dl * (float)v;
    }
  } else if constexpr (TT == TT_Q2_K) {  // quant_dequant.zig:892-919
    const uint8_t* blk = src + (v0 / 256) * 84;
    const int e0 = (int)(v0 % 256), g = e0 / 16;
    const float dl = h2f(ld16b(blk + 80)) * (float)(blk[g] & 15);
    const float ml = h2f(ld16b(blk + 82)) * (float)(blk[g] >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + i, k = e / 128, j = (e % 128) / 32, l = e % 32;
      o[i] = dl * (float)((blk[16 + 32 * k + l] >> (2 * j)) & 3u) - ml;
    }
  } else if constexpr (TT == TT_IQ4_XS) {  // quant_dequant.zig:324-345
    const uint8_t* blk = src + (v0 / 256) * 136;
    const int e0 = (int)(v0 % 256), ib = e0 / 32;
    const uint32_t sh = ld16b(blk + 2);
    const int ls = (int)(((blk[4 + ib / 2] >> (4 * (ib % 2))) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
    const float dl = h2f(ld16b(blk)) * (float)(ls - 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int j = (e0 + i) % 32;
      const uint32_t q = blk[8 + 16 * ib + (j & 15)];
      o[i] = dl * (float)iq4_value(j < 16 ? (q & 15u) : (q >> 4));
    }
  } else if constexpr (iq3(TT)) {
    // the four values are one grid entry: group k of sub-block ib
    // (IQ3_XXS quant_dequant.zig:417-445: db = d * (0.5 + ls) * 0.5;
    //  IQ3_S :362-415: db = d * (1 + 2 ls); value = (db * g) * (+-1))
    constexpr int BB = TT == TT_IQ3_XXS ? 98 : 110;
    const uint8_t* blk = src + (v0 / 256) * BB;
    const int e0 = (int)(v0 % 256), ib = e0 / 32, k = (e0 % 32) / 4;
    const float d = h2f(ld16b(blk));
    uint32_t e, s8;
    float db;
    if constexpr (TT == TT_IQ3_XXS) {
      const uint32_t aux = ld16b(blk + 66 + 4 * ib) | (ld16b(blk + 68 + 4 * ib) << 16);
      e = kIq3xxsGrid[blk[2 + 8 * ib + k]];
      s8 = iq_sign8((aux >> (7 * (k >> 1))) & 127u);
      db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
    } else {
      e = kIq3sGrid[blk[2 + 8 * ib + k] | (((blk[66 + ib] >> k) & 1u) << 8)];
      s8 = blk[74 + 4 * ib + (k >> 1)];
      db = d * (float)(1 + 2 * (int)((blk[106 + ib / 2] >> (4 * (ib % 2))) & 15u));
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float g = (float)((e >> (8 * i)) & 255u);
      o[i] = db * g * (((s8 >> (4 * (k & 1) + i)) & 1u) ? -1.0f : 1.0f);
    }
  } else {  // Q6_K
    const uint8_t* blk = src + (v0 / 256) * 210;
    const int e0 = (int)(v0 % 256);
    const float d = h2f(ld16b(blk + 208));
    const float ds = d * (float)(int)(int8_t)blk[192 + e0 / 16];  // four values share a 16-group
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = e0 + i, h = e / 128, q = (e % 128) / 32, l = e % 32;
      uint32_t lo = blk[64 * h + 32 * (q & 1) + l];
      lo = q >= 2 ? (lo >> 4) : (lo & 15u);
      const uint32_t hb = (blk[128 + 32 * h + l] >> (2 * q)) & 3u;
      o[i] = ds * (float)((int)(lo | (hb << 4)) - 32);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[v0 + i] = o[i];
}

hipError_t launch_dequant(int ttype, const void* src, float* dst, long nvals, hipStream_t s) {
  if (nvals <= 0) return hipSuccess;
  const unsigned grid = (unsigned)((nvals / 4 + 255) / 256);
  const uint8_t* p = (const uint8_t*)src;
  return dispatch_type(ttype, [&](auto tt) {
    hipLaunchKernelGGL(k_dequant<decltype(tt)::value>, dim3(grid), dim3(256), 0, s, p, dst, nvals);
    return hipGetLastError();
  });
}

}  // namespace qhip
