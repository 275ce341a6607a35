// gemv.hip -- batch-1 (and small-batch) quantized matrix-vector product.
//
// out[t*rows + r] = W[r] . xq[t]   (reference contract: src/backend.zig:177-178,
// src/kernels/cuda/api.h:104-112)
//
// Mapping.  A team of TPR consecutive lanes owns one weight row; lane j of the
// team walks the row's 64-value units j, j+TPR, j+2*TPR, ... loading each
// unit's bytes straight from HBM (dword-aligned 16/4-byte loads; each lane's
// span is at most 68 bytes, which measured at full stream bandwidth on MI355X)
// and the matching activation unit from L1/L2.  The team's float partials are
// folded with an xor-butterfly; lane 0 of the team stores.  NT tokens share
// each weight load (small-batch decode / the GEMV side of the MMQ crossover).
//
// Workgroups hold 4 waves; waves are independent (no barriers, no LDS).
#include "qhip_device.hpp"
#include "qhip_internal.hpp"

namespace qhip {

template <int TT, int TPR, int NT>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t* __restrict__ W,
                                               const uint8_t* __restrict__ XQ,
                                               float* __restrict__ Y, int rows, int upr,
                                               long row_bytes, long act_bytes, int tokens) {
  using U = Unit<TT>;
  constexpr int RPW = 64 / TPR;  // rows per wave
  const int lane = threadIdx.x & 63;
  const long row = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW + lane / TPR;
  const int j = lane % TPR;
  const bool active = row < rows;
  const uint8_t* wrow = W + (active ? row : 0) * row_bytes;
  for (int t0 = 0; t0 < tokens; t0 += NT) {
    float acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = 0.0f;
    if (active) {
#pragma unroll 2
      for (int u = j; u < upr; u += TPR) {
        const typename U::W w = U::load_w(wrow, u);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (NT == 1 || t0 + t < tokens) {
            const typename U::A a = U::load_a(XQ + (long)(t0 + t) * act_bytes, u);
            acc[t] += U::dot(w, a);
          }
        }
      }
    }
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) {
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] += __shfl_xor(acc[t], off, 64);
    }
    if (active && j == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
        if (NT == 1 || t0 + t < tokens) Y[(long)(t0 + t) * rows + row] = acc[t];
    }
  }
}

// Exact per-block integers, through the same unit decode as k_gemv.  One
// thread per (token, row, block-group): a 2-block unit for Q8_0 / IQ4_NL, a
// whole super-block (four units summed) for Q4_K / Q6_K.
// Layout of `ints`: [tokens][rows][nints]; nints = blocks per row, or
// 2 * super-blocks for Q4_K (isum, summs).
template <int TT>
__global__ __launch_bounds__(256) void k_block_ints(const uint8_t* __restrict__ W,
                                                     const uint8_t* __restrict__ XQ,
                                                     int* __restrict__ ints, int rows, int groups,
                                                     long row_bytes, long act_bytes, int tokens) {
  using U = Unit<TT>;
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  const long total = (long)tokens * rows * groups;
  if (gid >= total) return;
  const int g = (int)(gid % groups);
  const long rt = gid / groups;
  const long row = rt % rows, t = rt / rows;
  const uint8_t* wrow = W + row * row_bytes;
  const uint8_t* arow = XQ + t * act_bytes;
  if constexpr (TT == TT_Q8_0 || TT == TT_IQ4_NL) {
    int out[2];
    U::ints(U::load_w(wrow, g), U::load_a(arow, g), out);
    int* o = ints + rt * (2L * groups) + 2 * g;
    o[0] = out[0];
    o[1] = out[1];
  } else {
    int acc[2] = {0, 0};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      int part[2] = {0, 0};
      U::ints(U::load_w(wrow, 4 * g + c), U::load_a(arow, 4 * g + c), part);
      acc[0] += part[0];
      acc[1] += part[1];
    }
    if constexpr (TT == TT_Q4_K) {
      int* o = ints + rt * (2L * groups) + 2 * g;
      o[0] = acc[0];
      o[1] = acc[1];
    } else {
      ints[rt * groups + g] = acc[0];
    }
  }
}

// ---- generic fallback: any alignment, byte loads, one thread per (token, row)
__device__ __forceinline__ uint32_t ldb16(const uint8_t* p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8); }

template <int TT>
__global__ __launch_bounds__(256) void k_gemv_generic(const uint8_t* __restrict__ W,
                                                       const uint8_t* __restrict__ XQ,
                                                       float* __restrict__ Y, int rows, int cols,
                                                       long row_bytes, long act_bytes, int tokens) {
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long)rows * tokens) return;
  const long row = gid % rows, t = gid / rows;
  const uint8_t* w = W + row * row_bytes;
  const uint8_t* a = XQ + t * act_bytes;
  float acc = 0.0f;
  if constexpr (TT == TT_Q8_0 || TT == TT_IQ4_NL) {
    constexpr int BB = TT == TT_Q8_0 ? 34 : 18;
    for (int b = 0; b < cols / 32; ++b, w += BB, a += 34) {
      int s = 0;
      for (int j = 0; j < 32; ++j) {
        int wv;
        if constexpr (TT == TT_Q8_0) {
          wv = (int8_t)w[2 + j];
        } else {
          const uint32_t q = w[2 + (j & 15)];
          const uint32_t nib = j < 16 ? (q & 15u) : (q >> 4);
          const uint32_t tab = nib < 4 ? IQ4_T0 : nib < 8 ? IQ4_T1 : nib < 12 ? IQ4_T2 : IQ4_T3;
          wv = sext8(tab >> (8 * (nib & 3)));
        }
        s += wv * (int)(int8_t)a[2 + j];
      }
      acc += h2f(ldb16(w)) * h2f(ldb16(a)) * (float)s;
    }
  } else if constexpr (TT == TT_Q4_K) {
    for (int b = 0; b < cols / 256; ++b, w += 144, a += 292) {
      int is = 0, sm = 0;
      for (int sb = 0; sb < 8; ++sb) {
        int sc, mn;
        const uint8_t* s12 = w + 4;
        if (sb < 4) {
          sc = s12[sb] & 63; mn = s12[sb + 4] & 63;
        } else {
          sc = (s12[sb + 4] & 15) | ((s12[sb - 4] >> 6) << 4);
          mn = (s12[sb + 4] >> 4) | ((s12[sb] >> 6) << 4);
        }
        int sub = 0;
        for (int l = 0; l < 32; ++l) {
          const uint8_t q = w[16 + 32 * (sb / 2) + l];
          sub += ((sb & 1) ? (q >> 4) : (q & 15)) * (int)(int8_t)a[4 + 32 * sb + l];
        }
        is += sc * sub;
        sm += mn * (sext16(ldb16(a + 260 + 4 * sb)) + sext16(ldb16(a + 262 + 4 * sb)));
      }
      float dy;
      const uint32_t db = ldb16(a) | (ldb16(a + 2) << 16);
      dy = __builtin_bit_cast(float, db);
      acc += (dy * h2f(ldb16(w))) * (float)is - (dy * h2f(ldb16(w + 2))) * (float)sm;
    }
  } else {
    for (int b = 0; b < cols / 256; ++b, w += 210, a += 292) {
      int isum = 0;
      for (int g = 0; g < 16; ++g) {
        int sub = 0;
        for (int l16 = 0; l16 < 16; ++l16) {
          const int e = 16 * g + l16, h = e / 128, q = (e % 128) / 32, l = e % 32;
          int lo = (q & 1) ? w[64 * h + 32 + l] : w[64 * h + l];
          lo = q >= 2 ? (lo >> 4) : (lo & 15);
          const int hb = (w[128 + 32 * h + l] >> (2 * q)) & 3;
          sub += ((lo | (hb << 4)) - 32) * (int)(int8_t)a[4 + e];
        }
        isum += (int)(int8_t)w[192 + g] * sub;
      }
      const uint32_t db = ldb16(a) | (ldb16(a + 2) << 16);
      acc += (h2f(ldb16(w + 208)) * __builtin_bit_cast(float, db)) * (float)isum;
    }
  }
  Y[t * rows + row] = acc;
}

// ---- launchers ----------------------------------------------------------------

template <int TT, int TPR, int NT>
static hipError_t launch_gemv_t(const GemvArgs& g, hipStream_t s) {
  constexpr int RPB = 4 * (64 / TPR);
  const unsigned grid = (unsigned)((g.rows + RPB - 1) / RPB);
  hipLaunchKernelGGL((k_gemv<TT, TPR, NT>), dim3(grid), dim3(256), 0, s, (const uint8_t*)g.w,
                     (const uint8_t*)g.xq, g.out, g.rows, g.cols / 64, g.row_bytes, g.act_bytes,
                     g.tokens);
  return hipGetLastError();
}

template <int TT, int NT>
static hipError_t launch_gemv_tpr(const GemvArgs& g, int tpr, hipStream_t s) {
  switch (tpr) {
    case 1: return launch_gemv_t<TT, 1, NT>(g, s);
    case 2: return launch_gemv_t<TT, 2, NT>(g, s);
    case 4: return launch_gemv_t<TT, 4, NT>(g, s);
    case 8: return launch_gemv_t<TT, 8, NT>(g, s);
    case 16: return launch_gemv_t<TT, 16, NT>(g, s);
    case 32: return launch_gemv_t<TT, 32, NT>(g, s);
    case 64: return launch_gemv_t<TT, 64, NT>(g, s);
    default: return hipErrorInvalidValue;
  }
}

template <int TT>
static hipError_t launch_gemv_type(const GemvArgs& g, int tpr, int nt, hipStream_t s) {
  switch (nt) {
    case 1: return launch_gemv_tpr<TT, 1>(g, tpr, s);
    case 2: return launch_gemv_tpr<TT, 2>(g, tpr, s);
    case 4: return launch_gemv_tpr<TT, 4>(g, tpr, s);
    case 8: return launch_gemv_tpr<TT, 8>(g, tpr, s);
    default: return hipErrorInvalidValue;
  }
}

// Lanes per row: the smallest power of two that both fills the machine
// (>= kTargetWaves waves) and keeps the units-per-lane split balanced.
int gemv_pick_tpr(int rows, int cols) {
  const int upr = cols / 64;
  constexpr double kTargetWaves = 2048.0;  // 8 per CU on 256 CUs
  int best = 64;
  double best_score = -1.0;
  for (int tpr = 1; tpr <= 64; tpr *= 2) {
    if (tpr > 1 && tpr / 2 >= upr) break;  // more lanes than units
    const int per_lane = (upr + tpr - 1) / tpr;
    const double balance = (double)upr / ((double)tpr * per_lane);
    const double waves = (double)rows * tpr / 64.0;
    const double fill = waves >= kTargetWaves ? 1.0 : waves / kTargetWaves;
    const double score = balance * fill;
    if (score > best_score + 1e-9) {
      best_score = score;
      best = tpr;
    }
  }
  return best;
}

int gemv_pick_nt(int tokens) { return tokens >= 8 ? 8 : tokens >= 4 ? 4 : tokens >= 2 ? 2 : 1; }

hipError_t launch_gemv(const GemvArgs& g, int tpr, int nt, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  if (tpr <= 0) tpr = gemv_pick_tpr(g.rows, g.cols);
  if (nt <= 0) nt = gemv_pick_nt(g.tokens);
  switch (g.ttype) {
    case TT_Q8_0: return launch_gemv_type<TT_Q8_0>(g, tpr, nt, s);
    case TT_IQ4_NL: return launch_gemv_type<TT_IQ4_NL>(g, tpr, nt, s);
    case TT_Q4_K: return launch_gemv_type<TT_Q4_K>(g, tpr, nt, s);
    case TT_Q6_K: return launch_gemv_type<TT_Q6_K>(g, tpr, nt, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemv_generic(const GemvArgs& g, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  const long n = (long)g.rows * g.tokens;
  const unsigned grid = (unsigned)((n + 255) / 256);
  const uint8_t* w = (const uint8_t*)g.w;
  const uint8_t* a = (const uint8_t*)g.xq;
  switch (g.ttype) {
    case TT_Q8_0: hipLaunchKernelGGL(k_gemv_generic<TT_Q8_0>, dim3(grid), dim3(256), 0, s, w, a, g.out, g.rows, g.cols, g.row_bytes, g.act_bytes, g.tokens); break;
    case TT_IQ4_NL: hipLaunchKernelGGL(k_gemv_generic<TT_IQ4_NL>, dim3(grid), dim3(256), 0, s, w, a, g.out, g.rows, g.cols, g.row_bytes, g.act_bytes, g.tokens); break;
    case TT_Q4_K: hipLaunchKernelGGL(k_gemv_generic<TT_Q4_K>, dim3(grid), dim3(256), 0, s, w, a, g.out, g.rows, g.cols, g.row_bytes, g.act_bytes, g.tokens); break;
    case TT_Q6_K: hipLaunchKernelGGL(k_gemv_generic<TT_Q6_K>, dim3(grid), dim3(256), 0, s, w, a, g.out, g.rows, g.cols, g.row_bytes, g.act_bytes, g.tokens); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_block_ints(const GemvArgs& g, int* ints, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  const uint8_t* w = (const uint8_t*)g.w;
  const uint8_t* a = (const uint8_t*)g.xq;
  const int groups = (g.ttype == TT_Q8_0 || g.ttype == TT_IQ4_NL) ? g.cols / 64 : g.cols / 256;
  const long n = (long)g.tokens * g.rows * groups;
  const unsigned grid = (unsigned)((n + 255) / 256);
  switch (g.ttype) {
    case TT_Q8_0: hipLaunchKernelGGL(k_block_ints<TT_Q8_0>, dim3(grid), dim3(256), 0, s, w, a, ints, g.rows, groups, g.row_bytes, g.act_bytes, g.tokens); break;
    case TT_IQ4_NL: hipLaunchKernelGGL(k_block_ints<TT_IQ4_NL>, dim3(grid), dim3(256), 0, s, w, a, ints, g.rows, groups, g.row_bytes, g.act_bytes, g.tokens); break;
    case TT_Q4_K: hipLaunchKernelGGL(k_block_ints<TT_Q4_K>, dim3(grid), dim3(256), 0, s, w, a, ints, g.rows, groups, g.row_bytes, g.act_bytes, g.tokens); break;
    case TT_Q6_K: hipLaunchKernelGGL(k_block_ints<TT_Q6_K>, dim3(grid), dim3(256), 0, s, w, a, ints, g.rows, groups, g.row_bytes, g.act_bytes, g.tokens); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace qhip
