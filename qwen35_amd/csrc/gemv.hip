// gemv.hip -- batch-1 (and small-batch) quantized matrix-vector product.
//
// out[t*rows + r] = W[r] . xq[t]   (reference contract: src/backend.zig:177-178,
// src/kernels/cuda/api.h:104-112)
//
// Mapping.  A team of S consecutive lanes owns NR consecutive weight rows
// (S = 1..64, any value; a wave holds floor(64/S) teams).  Lane j of the team
// walks the rows' 64-value units j, j+S, j+2S, ... (Unit<> in
// qhip_device.hpp); consecutive units are adjacent in memory, so each load
// instruction of a team reads one contiguous span of a row straight from HBM.
// The matching activation unit comes from L1/L2 once and serves all NR rows:
// activation bytes delivered to lanes, not HBM bytes, are what the texture
// path spends most of its time on, so NR > 1 cuts that traffic NR-fold.  The team's float partials are folded with a
// segmented shuffle tree whose order depends only on S, so results are
// deterministic.  Waves are independent: no LDS, no barriers, no atomics.
//
// S trades balance against parallelism: matrices with many rows use few
// lanes per row, matrices with few long rows (the FFN down projection) use
// many.  NT tokens share each weight unit held in registers (small-batch
// decode and the GEMV side of the GEMV-vs-MMQ crossover).
#include "qhip_device.hpp"
#include "qhip_internal.hpp"

namespace qhip {

template <int TT, int NT, int NR>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t* __restrict__ W,
                                               const uint8_t* __restrict__ XQ,
                                               float* __restrict__ Y, int rows, long row_bytes,
                                               long act_bytes, int upr, int team, int tokens) {
  using U = Unit<TT>;
  const int lane = threadIdx.x & 63;
  const int tpw = 64 / team;                       // teams per wave
  const int r = lane / team, j = lane - r * team;  // team index, lane in team
  // team r owns NR consecutive rows
  const long row0 = (((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * tpw + r) * NR;
  const bool active = r < tpw && row0 < rows;
  const uint8_t* wrow[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const long rk = row0 + k < rows ? row0 + k : rows - 1;  // tail rows re-read the last row
    wrow[k] = W + (active ? rk : 0) * row_bytes;
  }
  const int u_end = active ? upr : 0;
  for (int t0 = 0; t0 < tokens; t0 += NT) {
    float acc[NT][NR];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int k = 0; k < NR; ++k) acc[t][k] = 0.0f;
#pragma unroll 2
    for (int u = j; u < u_end; u += team) {
      typename U::W w[NR];
#pragma unroll
      for (int k = 0; k < NR; ++k) w[k] = U::load_w(wrow[k], u);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if (NT == 1 || t0 + t < tokens) {
          const typename U::A a = U::load_a(XQ + (long)(t0 + t) * act_bytes, u);
#pragma unroll
          for (int k = 0; k < NR; ++k) acc[t][k] += U::dot(w[k], a);
        }
      }
    }
    // segmented tree over the team: lane j adds lane j+off while j+off < S
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      if (off < team) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
          for (int k = 0; k < NR; ++k) {
            const float v = __shfl_down(acc[t][k], off, 64);
            if (j + off < team) acc[t][k] += v;
          }
      }
    }
    if (active && j == 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int k = 0; k < NR; ++k)
          if ((NT == 1 || t0 + t < tokens) && row0 + k < rows)
            Y[(long)(t0 + t) * rows + row0 + k] = acc[t][k];
    }
  }
}

// Exact per-block integers through the same unit decode as k_gemv.  One
// thread per (token, row, block group): a 2-block unit for Q8_0 / IQ4_NL, a
// whole super-block (its four units summed) for Q4_K / Q6_K.  Layout of
// `ints`: [tokens][rows][nints]; nints = blocks per row, or 2 per super-block
// for Q4_K (isum, summs).
template <int TT>
__global__ __launch_bounds__(256) void k_block_ints(const uint8_t* __restrict__ W,
                                                     const uint8_t* __restrict__ XQ,
                                                     int* __restrict__ ints, int rows, int groups,
                                                     long row_bytes, long act_bytes, int tokens) {
  using U = Unit<TT>;
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long)tokens * rows * groups) return;
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
      const float dy = __builtin_bit_cast(float, ldb16(a) | (ldb16(a + 2) << 16));
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
      const float dy = __builtin_bit_cast(float, ldb16(a) | (ldb16(a + 2) << 16));
      acc += (h2f(ldb16(w + 208)) * dy) * (float)isum;
    }
  }
  Y[t * rows + row] = acc;
}

// ---- launch shape and launchers --------------------------------------------------

// Lanes per row: score each team size by lane utilisation (idle lanes in a
// wave, uneven unit split) times machine fill (waves relative to
// target_waves), preferring fewer lanes per row unless a larger team is
// clearly better.
int gemv_pick_team(int rows, int cols, int target_waves) {
  const int units = cols / 64;
  int best = 1;
  double best_score = -1.0;
  for (int s = 1; s <= 64 && s <= units; ++s) {
    const int per_lane = (units + s - 1) / s;
    const int rpw = 64 / s;
    const double util = (double)(rpw * s) / 64.0 * (double)units / ((double)s * per_lane);
    const double waves = (double)(rows + rpw - 1) / rpw;
    const double fill = waves >= target_waves ? 1.0 : waves / target_waves;
    const double score = util * fill;
    if (score > best_score * 1.02) {
      best_score = score;
      best = s;
    }
  }
  return best;
}

int gemv_pick_nt(int tokens) { return tokens >= 8 ? 8 : tokens >= 4 ? 4 : tokens >= 2 ? 2 : 1; }

template <int TT, int NT, int NR>
static hipError_t launch_gemv_t(const GemvArgs& g, int team, hipStream_t s) {
  const int upr = g.cols / 64;
  if (team > upr) team = upr;
  if (team > 64) team = 64;
  const int tpw = 64 / team;
  const long teams = (g.rows + NR - 1) / NR;
  const long waves = (teams + tpw - 1) / tpw;
  const unsigned grid = (unsigned)((waves + 3) / 4);
  hipLaunchKernelGGL((k_gemv<TT, NT, NR>), dim3(grid), dim3(256), 0, s, (const uint8_t*)g.w,
                     (const uint8_t*)g.xq, g.out, g.rows, g.row_bytes, g.act_bytes, upr, team,
                     g.tokens);
  return hipGetLastError();
}

template <int TT, int NT>
static hipError_t launch_gemv_nr(const GemvArgs& g, int team, int nr, hipStream_t s) {
  switch (nr) {
    case 1: return launch_gemv_t<TT, NT, 1>(g, team, s);
    case 2: return launch_gemv_t<TT, NT, 2>(g, team, s);
    case 4: return launch_gemv_t<TT, NT, 4>(g, team, s);
    default: return hipErrorInvalidValue;
  }
}

template <int TT>
static hipError_t launch_gemv_type(const GemvArgs& g, int team, int nt, int nr, hipStream_t s) {
  switch (nt) {
    case 1: return launch_gemv_nr<TT, 1>(g, team, nr, s);
    case 2: return launch_gemv_nr<TT, 2>(g, team, nr > 2 ? 2 : nr, s);
    case 4: return launch_gemv_t<TT, 4, 1>(g, team, s);
    case 8: return launch_gemv_t<TT, 8, 1>(g, team, s);
    default: return hipErrorInvalidValue;
  }
}

// Default launch shape for batch-1, from sweeps on MI355X at the benchmark
// shapes: Q6_K decode issues the most loads per byte and wants the most
// parallelism (one row per lane group of up to 64 lanes); Q4_K and IQ4_NL
// want the activation reused over two rows per lane; Q8_0 over two rows
// when the matrix is large enough to fill the GPU anyway.
static void default_shape(const GemvArgs& g, int& team, int& nr) {
  const int upr = g.cols / 64;
  switch (g.ttype) {
    case TT_Q6_K: nr = 1; team = 64; break;
    case TT_Q4_K: nr = g.rows >= 16384 && upr <= 40 ? 4 : 2; team = upr <= 40 ? 40 : 20; break;
    case TT_IQ4_NL: nr = 2; team = 20; break;
    default: nr = g.rows >= 4096 ? 2 : 1; team = 16; break;
  }
  if (team > upr) team = upr;
  // small matrices: fall back to one row per lane and the fill-based team
  const long waves = ((long)(g.rows + nr - 1) / nr + 64 / team - 1) / (64 / team);
  if (waves < kGemvTargetWaves / 2 && nr > 1) {
    nr = 1;
    team = gemv_pick_team(g.rows, g.cols, kGemvTargetWaves);
  }
}

hipError_t launch_gemv(const GemvArgs& g, int team, int nt, int nr, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  if (team <= 0 && nr <= 0 && g.tokens == 1) {
    default_shape(g, team, nr);
  } else {
    if (nr <= 0) nr = 1;
    if (team <= 0) team = gemv_pick_team((g.rows + nr - 1) / nr, g.cols, kGemvTargetWaves);
  }
  if (nt <= 0) nt = gemv_pick_nt(g.tokens);
  switch (g.ttype) {
    case TT_Q8_0: return launch_gemv_type<TT_Q8_0>(g, team, nt, nr, s);
    case TT_IQ4_NL: return launch_gemv_type<TT_IQ4_NL>(g, team, nt, nr, s);
    case TT_Q4_K: return launch_gemv_type<TT_Q4_K>(g, team, nt, nr, s);
    case TT_Q6_K: return launch_gemv_type<TT_Q6_K>(g, team, nt, nr, s);
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

template <int TT>
static hipError_t launch_ints_t(const GemvArgs& g, int* ints, hipStream_t s) {
  const int groups = (TT == TT_Q8_0 || TT == TT_IQ4_NL) ? g.cols / 64 : g.cols / 256;
  const long n = (long)g.tokens * g.rows * groups;
  const unsigned grid = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(k_block_ints<TT>, dim3(grid), dim3(256), 0, s, (const uint8_t*)g.w,
                     (const uint8_t*)g.xq, ints, g.rows, groups, g.row_bytes, g.act_bytes, g.tokens);
  return hipGetLastError();
}

hipError_t launch_block_ints(const GemvArgs& g, int* ints, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  switch (g.ttype) {
    case TT_Q8_0: return launch_ints_t<TT_Q8_0>(g, ints, s);
    case TT_IQ4_NL: return launch_ints_t<TT_IQ4_NL>(g, ints, s);
    case TT_Q4_K: return launch_ints_t<TT_Q4_K>(g, ints, s);
    case TT_Q6_K: return launch_ints_t<TT_Q6_K>(g, ints, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qhip
