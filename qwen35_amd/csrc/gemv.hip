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

template <int TT, int NT, int NR, bool IMG = false, int WPB = 4>
__global__ __launch_bounds__(64 * WPB) void k_gemv(const uint8_t* __restrict__ W,
                                               const uint8_t* __restrict__ XQ,
                                               float* __restrict__ Y, int rows, long row_bytes,
                                               long act_bytes, int upr, int team, int tokens) {
  using U = Unit<TT>;
  grid_prologue<TT>();
  const int lane = threadIdx.x & 63;
  const int tpw = 64 / team;                       // teams per wave
  const int r = lane / team, j = lane - r * team;  // team index, lane in team
  // team r owns NR consecutive rows
  const long row0 = (((long)blockIdx.x * WPB + (threadIdx.x >> 6)) * tpw + r) * NR;
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
    for (int u = j; u < u_end; u += team) {
      typename U::W w[NR];
#pragma unroll
      for (int k = 0; k < NR; ++k) w[k] = load_unit<TT, IMG>(wrow[k], u, upr);
      if constexpr (NT == 1) {
        const typename U::A a = U::load_a(XQ + (long)t0 * act_bytes, u);
        // the unit's loads before its dots, as in k_gemv_mw, for the formats
        // it helps (Q8_0 [17408, 5120] 23.4 against 31.9 us; Q6_K image
        // [19456, 2560] 64 lanes x 2 rows 10.3 against 12.1, [17408, 5120]
        // 20 x 2 16.9 against 19.1; Q4_K [19456, 2560] 40 x 4 8.1 against
        // 8.3; IQ3_XXS 12.1-12.9 against 13.2); the others keep the
        // compiler's order (IQ4_NL [17408, 5120] 15.3 against 19.2 with it;
        // Q2_K, IQ4_XS, IQ3_S 1-2% slower)
        if constexpr (TT == TT_Q8_0 || TT == TT_Q4_K || TT == TT_Q6_K || TT == TT_IQ3_XXS)
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < NR; ++k) acc[0][k] += U::dot(w[k], a);
      } else {
        // decode each weight unit once, multiply it by every token of the pass
        typename Prep<TT>::P p[NR];
#pragma unroll
        for (int k = 0; k < NR; ++k) p[k] = Prep<TT>::prep(w[k]);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          if (t0 + t < tokens) {
            const typename U::A a = U::load_a(XQ + (long)(t0 + t) * act_bytes, u);
#pragma unroll
            for (int k = 0; k < NR; ++k) acc[t][k] += Prep<TT>::dotp(p[k], a);
          }
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

// Teams of WV whole waves (128 or 256 lanes per row group), one token.  For
// matrices with few long rows (the FFN down projection): the rows' units are
// split over the team's waves, so NR rows can share each activation load
// without cutting the number of waves in flight.  Wave s of a team walks
// units lane + 64s, stepping 64*WV; each wave folds its lanes by DPP
// (wave_sum_to_lane63), then the team's waves are added in wave order
// through LDS (deterministic).
template <int TT, int NR, int WV, bool IMG = false>
__global__ __launch_bounds__(256) void k_gemv_mw(const uint8_t* __restrict__ W,
                                                  const uint8_t* __restrict__ XQ,
                                                  float* __restrict__ Y, int rows, long row_bytes,
                                                  int upr) {
  using U = Unit<TT>;
  grid_prologue<TT>();
  constexpr int TPB = 4 / WV;  // teams per workgroup
  __shared__ float part[4][NR];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int tm = wv / WV, sl = wv % WV;
  const long row0 = ((long)blockIdx.x * TPB + tm) * NR;
  const bool active = row0 < rows;
  const uint8_t* wrow[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const long rk = row0 + k < rows ? row0 + k : rows - 1;
    wrow[k] = W + (active ? rk : 0) * row_bytes;
  }
  const int u_end = active ? upr : 0;
  float acc[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) acc[k] = 0.0f;
  for (int u = lane + 64 * sl; u < u_end; u += 64 * WV) {
    typename U::W w[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) w[k] = load_unit<TT, IMG>(wrow[k], u, upr);
    const typename U::A a = U::load_a(XQ, u);
    // every load of the unit is issued before the first dot: left to itself
    // the scheduler sinks some of them between the dots to save registers,
    // and each such load then costs the wave a memory round trip of its own
    // (Q6_K [5120, 17408] from the K-quant image, two rows per four-wave
    // team: 16.7 us against 22.7; [2560, 9728] 6.05 against 6.61; Q4_K
    // [17408, 5120] from the GGUF rows 11.3 against 11.8)
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < NR; ++k) acc[k] += U::dot(w[k], a);
  }
#pragma unroll
  for (int k = 0; k < NR; ++k) acc[k] = wave_sum_to_lane63(acc[k]);
  if (lane == 63) {
#pragma unroll
    for (int k = 0; k < NR; ++k) part[wv][k] = acc[k];
  }
  __syncthreads();
  if (sl == 0 && lane < NR && active && row0 + lane < rows) {
    float v = part[tm * WV][lane];
#pragma unroll
    for (int q = 1; q < WV; ++q) v += part[tm * WV + q][lane];
    Y[row0 + lane] = v;
  }
}

// Balanced teams of WV whole waves (1, 2 or 4) owning NR rows of 64a + b
// units (1 <= a <= A WV, NR b <= 64 WV), one token, every load of a lane
// issued before its first dot.  Wave s takes the whole rounds r = s, s + WV,
// ... (unit lane + 64 r of each of the NR rows, one activation unit shared by
// them); the NR b tail pairs (row, unit) of the team go one per lane, pair
// t = WV lane + s to row t / b, unit 64 a + t % b, with an activation unit of
// its own.  k_gemv_mw gives the tail units to the first b lanes, which then
// make a second round trip for the NR rows while the rest of the team idles.
// The partials fold as in k_gemv_mw (deterministic).
template <int TT, int NR, int WV, int A, bool IMG = false>
__global__ __launch_bounds__(256) void k_gemv_bal(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ,
                                                   float* __restrict__ Y, int rows, long row_bytes, int upr) {
  using U = Unit<TT>;
  constexpr int TPB = 4 / WV;  // teams per workgroup
  __shared__ float part[4][NR];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int tm = wv / WV, sl = wv % WV;
  const long row0 = ((long)blockIdx.x * TPB + tm) * NR;
  const bool active = row0 < rows;
  const int a = upr >> 6, b = upr & 63;
  const int t = lane * WV + sl;
  const bool tail = active && t < NR * b;
  const int tk = tail ? t / b : 0;
  float acc[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) acc[k] = 0.0f;
  if (active) {
    const uint8_t* wrow[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) wrow[k] = W + (row0 + k < rows ? row0 + k : rows - 1) * row_bytes;
    typename U::W w[A][NR];
    typename U::A x[A];
#pragma unroll
    for (int i = 0; i < A; ++i) {
      if (sl + WV * i < a) {
        const int u = lane + 64 * (sl + WV * i);
#pragma unroll
        for (int k = 0; k < NR; ++k) w[i][k] = load_unit<TT, IMG>(wrow[k], u, upr);
        x[i] = U::load_a(XQ, u);
      }
    }
    typename U::W wt;
    typename U::A xt;
    if (tail) {
      const int u = 64 * a + (t - tk * b);
      wt = load_unit<TT, IMG>(W + (row0 + tk < rows ? row0 + tk : rows - 1) * row_bytes, u, upr);
      xt = U::load_a(XQ, u);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < A; ++i) {
      if (sl + WV * i < a) {
#pragma unroll
        for (int k = 0; k < NR; ++k) acc[k] += U::dot(w[i][k], x[i]);
      }
    }
    if (tail) {
      const float v = U::dot(wt, xt);
#pragma unroll
      for (int k = 0; k < NR; ++k)
        if (k == tk) acc[k] += v;
    }
  }
#pragma unroll
  for (int k = 0; k < NR; ++k) acc[k] = wave_sum_to_lane63(acc[k]);
  if (lane == 63) {
#pragma unroll
    for (int k = 0; k < NR; ++k) part[wv][k] = acc[k];
  }
  __syncthreads();
  if (sl == 0 && lane < NR && active && row0 + lane < rows) {
    float v = part[tm * WV][lane];
#pragma unroll
    for (int q = 1; q < WV; ++q) v += part[tm * WV + q][lane];
    Y[row0 + lane] = v;
  }
}

// ---- quantize + GEMV in one launch (batch 1) ---------------------------------------
// Every workgroup quantizes the f32 activation itself, bit-exactly as the
// standalone quantizers do, into an LDS image split into planes (ActSplit:
// int8 values, per-block f32 scales, Q8_K 16-value sums), then runs the same
// team-of-lanes GEMV as k_gemv with the activation read from LDS instead of
// through the texture path.  Before quantizing, each lane issues the loads of
// its first weight unit, so the quantize prologue runs while those bytes are
// on their way from HBM; later units are prefetched one ahead.  This removes
// the separate quantize launch (about 2-3 us each on this GPU) from every
// decode matvec.  Workgroup 0 also writes the quantized activation in the
// reference layout when `XQ` is not null.
__host__ __device__ constexpr long fused_lds_qs(int cols) { return (long)cols / 64 * kSplitUnit; }
__host__ __device__ constexpr long fused_lds_bytes(int ttype, int cols) {
  // qs (80 B per 64 values) | d[nblk] f32 (16-aligned) | Q8_K: bs[cols/16] int16
  return act32(ttype)
             ? fused_lds_qs(cols) + (((long)cols / 32 * 4 + 15) & ~15L)
             : fused_lds_qs(cols) + (((long)cols / 256 * 4 + 15) & ~15L) + (long)cols / 16 * 2;
}

//
// Split-K form (SK): the rows' units are cut into slices of `slice_units`
// (whole super-blocks); workgroup column blockIdx.y owns slice blockIdx.y of
// the rows of its row tile blockIdx.x and quantizes only that slice of x, so
// a long activation is quantized once per row tile rather than once per
// row group.  Each workgroup writes its partial sums to part[slice][row];
// the last workgroup of a row tile to finish (counted by an atomic in
// cnt[tile]) adds the partials in slice order, writes y and puts the counter
// back to zero, so the result does not depend on completion order.  No
// workgroup waits for another: the last one to arrive does the sum.
template <int TT, int NR, int WGS, bool SK = false>
__global__ __launch_bounds__(WGS) void k_gemv_q(const uint8_t* __restrict__ W, const float* __restrict__ X,
                                                 uint8_t* __restrict__ XQ, float* __restrict__ Y, int rows,
                                                 int cols, long row_bytes, int upr, int team,
                                                 float* __restrict__ part, unsigned* __restrict__ cnt,
                                                 int slice_units, long slice_wbytes) {
  using U = Unit<TT>;
  grid_prologue<TT>();
  constexpr bool K32 = act32(TT);
  if constexpr (SK) {
    const int u0 = (int)blockIdx.y * slice_units;
    X += 64L * u0;
    W += (long)blockIdx.y * slice_wbytes;
    if (XQ) XQ += K32 ? 68L * u0 : 73L * u0;  // 2 x 34 B per unit (Q8_0), 292 B per 4 units (Q8_K)
    upr = min(slice_units, upr - u0);
    cols = 64 * upr;
  }
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int nblk = K32 ? cols / 32 : cols / 256;
  uint8_t* qs = lds;
  const int qsb = (int)fused_lds_qs(cols);
  float* dsc = (float*)(lds + qsb);
  int16_t* bs = (int16_t*)(lds + qsb + ((nblk * 4 + 15) & ~15));
  const ActSplit sp{qs, dsc, bs};

  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int tpw = 64 / team;
  const int r = lane / team, j = lane - r * team;
  const long row0 = (((long)blockIdx.x * (WGS / 64) + wv) * tpw + r) * NR;
  const bool active = r < tpw && row0 < rows;
  const uint8_t* wrow[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) {
    const long rk = row0 + k < rows ? row0 + k : rows - 1;
    wrow[k] = W + (active ? rk : 0) * row_bytes;
  }
  const int u_end = active ? upr : 0;

  // The activation loads of the first RX quantize rounds are issued before
  // the first weight unit's: loads complete in order, so the quantize can
  // start as soon as x arrives instead of after the weights.
  constexpr int RX = 4;
  constexpr int STEP = K32 ? WGS / 32 : WGS / 64;  // blocks per round
  const bool out_q = XQ != nullptr && blockIdx.x == 0;
  float xs[RX];
  float4 xf[RX];
#pragma unroll
  for (int rd = 0; rd < RX; ++rd) {
    if constexpr (K32) {
      const int b = rd * STEP + (threadIdx.x >> 5);
      xs[rd] = b < nblk ? X[32 * b + (threadIdx.x & 31)] : 0.0f;
    } else {
      const int b = rd * STEP + wv;
      xf[rd] = b < nblk ? *(const float4*)(X + 256L * b + 4 * lane) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }

  typename U::W wcur[NR];
  if (j < u_end) {
#pragma unroll
    for (int k = 0; k < NR; ++k) wcur[k] = U::load_w(wrow[k], j);
  }

  // one quantize round: block b from the value(s) v
  auto quant32 = [&](int b, float v) {
    const int i = threadIdx.x & 31;
    const bool ok = b < nblk;
    uint32_t hb;
    const int q = quant_q8_0_lane(v, hb);
    if (ok) {
      qs[split_off(32 * b + i)] = (uint8_t)(int8_t)q;
      if (i == 0) dsc[b] = h2f(hb);
      if (out_q) {
        uint8_t* ob = XQ + 34L * b;
        ob[2 + i] = (uint8_t)(int8_t)q;
        if (i == 0) {
          ob[0] = (uint8_t)hb;
          ob[1] = (uint8_t)(hb >> 8);
        }
      }
    }
  };
  auto quant256 = [&](int b, float4 f) {
    const bool ok = b < nblk;
    float v[4] = {f.x, f.y, f.z, f.w};
    int gsum;
    float scale;
    const uint32_t packed = quant_q8_K_lane(v, gsum, scale);
    if (ok) {
      *(uint32_t*)(qs + split_off(256 * b + 4 * lane)) = packed;
      if ((lane & 3) == 0) bs[16 * b + (lane >> 2)] = (int16_t)gsum;
      if (lane == 0) dsc[b] = scale;
      if (out_q) {
        uint8_t* ob = XQ + 292L * b;
        *(uint32_t*)(ob + 4 + 4 * lane) = packed;
        if ((lane & 3) == 0) *(int16_t*)(ob + 260 + 2 * (lane >> 2)) = (int16_t)gsum;
        if (lane == 0) *(float*)ob = scale;
      }
    }
  };
  // K32: one value per thread, a 32-lane group per block; else a wave per
  // 256-value block, four values per lane.  Rounds are uniform over the
  // workgroup (every lane takes part in the shuffles).
#pragma unroll
  for (int rd = 0; rd < RX; ++rd) {
    if (rd * STEP < nblk) {
      if constexpr (K32) quant32(rd * STEP + (threadIdx.x >> 5), xs[rd]);
      else quant256(rd * STEP + wv, xf[rd]);
    }
  }
  for (int b0 = RX * STEP; b0 < nblk; b0 += STEP) {
    if constexpr (K32) {
      const int b = b0 + (threadIdx.x >> 5);
      quant32(b, b < nblk ? X[32 * b + (threadIdx.x & 31)] : 0.0f);
    } else {
      const int b = b0 + wv;
      quant256(b, b < nblk ? *(const float4*)(X + 256L * b + 4 * lane) : make_float4(0.0f, 0.0f, 0.0f, 0.0f));
    }
  }
  __syncthreads();

  float acc[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) acc[k] = 0.0f;
  for (int u = j; u < u_end; u += team) {
    const int un = u + team;
    typename U::W wnext[NR];
    if (un < u_end) {
#pragma unroll
      for (int k = 0; k < NR; ++k) wnext[k] = U::load_w(wrow[k], un);
    }
    const typename U::A a = U::load_a_split(sp, u);
#pragma unroll
    for (int k = 0; k < NR; ++k) acc[k] += U::dot(wcur[k], a);
#pragma unroll
    for (int k = 0; k < NR; ++k) wcur[k] = wnext[k];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    if (off < team) {
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const float v = __shfl_down(acc[k], off, 64);
        if (j + off < team) acc[k] += v;
      }
    }
  }
  if constexpr (!SK) {
    if (active && j == 0) {
#pragma unroll
      for (int k = 0; k < NR; ++k)
        if (row0 + k < rows) Y[row0 + k] = acc[k];
    }
  } else {
    // deterministic hand-off (sk_* in qhip_device.hpp): partials in
    // part[slice][row], the last workgroup of the row tile adds them in
    // slice order
    float* pp = part + (long)blockIdx.y * rows;
    if (active && j == 0) {
#pragma unroll
      for (int k = 0; k < NR; ++k)
        if (row0 + k < rows) sk_store(pp + row0 + k, acc[k]);
    }
    if (sk_arrive(cnt + blockIdx.x, gridDim.y)) {
      const int rpw = (WGS / 64) * tpw * NR;
      const int ns = (int)gridDim.y;
      for (int i = threadIdx.x; i < rpw; i += WGS) {
        const long rr = (long)blockIdx.x * rpw + i;
        if (rr < rows) {
          float v = 0.0f;
          int q = 0;
          for (; q + 8 <= ns; q += 8) {
            float t[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) t[c] = sk_load(part + (long)(q + c) * rows + rr);
#pragma unroll
            for (int c = 0; c < 8; ++c) v += t[c];
          }
          for (; q < ns; ++q) v += sk_load(part + (long)q * rows + rr);
          Y[rr] = v;
        }
      }
      sk_reset(cnt + blockIdx.x);
    }
  }
}

// Exact per-block integers through the same unit decode as k_gemv.  One
// thread per (token, row, block group): a unit of two 32-value blocks for the
// 32-value formats and IQ4_XS (whose integers are per 32-value block), a whole
// super-block (its four units summed) for the other K-quants.  Layout of
// `ints`: [tokens][rows][nints]; nints = 32-value blocks per row (twice that
// for Q4_1: sumi, sumy per block), or per super-block 2 (isum, summs: Q4_K,
// Q5_K, Q2_K) or 1 (Q6_K, Q3_K).
constexpr bool per_block_ints(int tt) { return act32(tt) || tt == TT_IQ4_XS || iq3(tt); }

template <int TT>
__global__ __launch_bounds__(256) void k_block_ints(const uint8_t* __restrict__ W,
                                                     const uint8_t* __restrict__ XQ,
                                                     int* __restrict__ ints, int rows, int groups,
                                                     long row_bytes, long act_bytes, int tokens) {
  using U = Unit<TT>;
  grid_prologue<TT>();
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= (long)tokens * rows * groups) return;
  const int g = (int)(gid % groups);
  const long rt = gid / groups;
  const long row = rt % rows, t = rt / rows;
  const uint8_t* wrow = W + row * row_bytes;
  const uint8_t* arow = XQ + t * act_bytes;
  if constexpr (per_block_ints(TT)) {
    constexpr int NI = U::kInts;
    int out[NI];
    U::ints(U::load_w(wrow, g), U::load_a(arow, g), out);
    int* o = ints + rt * ((long)NI * groups) + NI * g;
#pragma unroll
    for (int i = 0; i < NI; ++i) o[i] = out[i];
  } else {
    int acc[2] = {0, 0};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      int part[2] = {0, 0};
      U::ints(U::load_w(wrow, 4 * g + c), U::load_a(arow, 4 * g + c), part);
      acc[0] += part[0];
      acc[1] += part[1];
    }
    if constexpr (U::kInts == 2) {
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
  if constexpr (act32(TT)) {
    constexpr int BB = blk32_bytes(TT), QO = TT == TT_Q4_1 ? 4 : 2;
    for (int b = 0; b < cols / 32; ++b, w += BB, a += 34) {
      int s = 0, sy = 0;
      for (int j = 0; j < 32; ++j) {
        int wv;
        if constexpr (TT == TT_Q8_0) {
          wv = (int8_t)w[2 + j];
        } else {
          const uint32_t q = w[QO + (j & 15)];
          const uint32_t nib = j < 16 ? (q & 15u) : (q >> 4);
          if constexpr (TT == TT_IQ4_NL) {
            const uint32_t tab = nib < 4 ? IQ4_T0 : nib < 8 ? IQ4_T1 : nib < 12 ? IQ4_T2 : IQ4_T3;
            wv = sext8(tab >> (8 * (nib & 3)));
          } else {
            wv = TT == TT_Q4_0 ? (int)nib - 8 : (int)nib;
          }
        }
        s += wv * (int)(int8_t)a[2 + j];
        sy += (int)(int8_t)a[2 + j];
      }
      const float dy = h2f(ldb16(a));
      acc += h2f(ldb16(w)) * dy * (float)s;
      if constexpr (TT == TT_Q4_1) acc += h2f(ldb16(w + 2)) * dy * (float)sy;
    }
  } else {
    constexpr int BB = TT == TT_Q4_K ? 144 : TT == TT_Q6_K ? 210 : TT == TT_Q5_K ? 176 : TT == TT_Q3_K ? 110
                     : TT == TT_Q2_K ? 84 : TT == TT_IQ3_XXS ? 98 : TT == TT_IQ3_S ? 110 : 136;
    for (int b = 0; b < cols / 256; ++b, w += BB, a += 292) {
      const float dy = __builtin_bit_cast(float, ldb16(a) | (ldb16(a + 2) << 16));
      const int8_t* q8 = (const int8_t*)(a + 4);
      if constexpr (TT == TT_Q4_K || TT == TT_Q5_K) {
        constexpr int QS = TT == TT_Q4_K ? 16 : 48;
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
            const uint8_t q = w[QS + 32 * (sb / 2) + l];
            int v = (sb & 1) ? (q >> 4) : (q & 15);
            if constexpr (TT == TT_Q5_K) v |= ((w[16 + l] >> sb) & 1) << 4;
            sub += v * (int)q8[32 * sb + l];
          }
          is += sc * sub;
          sm += mn * (sext16(ldb16(a + 260 + 4 * sb)) + sext16(ldb16(a + 262 + 4 * sb)));
        }
        acc += (dy * h2f(ldb16(w))) * (float)is - (dy * h2f(ldb16(w + 2))) * (float)sm;
      } else if constexpr (TT == TT_Q6_K) {
        int isum = 0;
        for (int g = 0; g < 16; ++g) {
          int sub = 0;
          for (int l16 = 0; l16 < 16; ++l16) {
            const int e = 16 * g + l16, h = e / 128, q = (e % 128) / 32, l = e % 32;
            int lo = (q & 1) ? w[64 * h + 32 + l] : w[64 * h + l];
            lo = q >= 2 ? (lo >> 4) : (lo & 15);
            const int hb = (w[128 + 32 * h + l] >> (2 * q)) & 3;
            sub += ((lo | (hb << 4)) - 32) * (int)q8[e];
          }
          isum += (int)(int8_t)w[192 + g] * sub;
        }
        acc += (h2f(ldb16(w + 208)) * dy) * (float)isum;
      } else if constexpr (TT == TT_Q3_K) {
        uint32_t u[3];
        for (int i = 0; i < 3; ++i)
          u[i] = (uint32_t)w[96 + 4 * i] | ((uint32_t)w[97 + 4 * i] << 8) | ((uint32_t)w[98 + 4 * i] << 16) |
                 ((uint32_t)w[99 + 4 * i] << 24);
        int isum = 0;
        for (int g = 0; g < 16; ++g) {
          const int c = g / 4, k = g % 4;
          const uint32_t base = (c & 1) ? u[1] : u[0];
          const uint32_t scw = ((c >= 2 ? (base >> 4) : base) & 0x0F0F0F0Fu) | (((u[2] >> (2 * c)) & 0x03030303u) << 4);
          const int sc = (int)((scw >> (8 * k)) & 0xFFu) - 32;
          int sub = 0;
          for (int l16 = 0; l16 < 16; ++l16) {
            const int e = 16 * g + l16, h = e / 128, j = (e % 128) / 32, l = e % 32;
            const int v = ((w[32 + 32 * h + l] >> (2 * j)) & 3) - (((w[l] >> (4 * h + j)) & 1) ? 0 : 4);
            sub += v * (int)q8[e];
          }
          isum += sc * sub;
        }
        acc += (h2f(ldb16(w + 108)) * dy) * (float)isum;
      } else if constexpr (TT == TT_Q2_K) {
        int isum = 0, summs = 0;
        for (int g = 0; g < 16; ++g) {
          int sub = 0;
          for (int l16 = 0; l16 < 16; ++l16) {
            const int e = 16 * g + l16, k = e / 128, j = (e % 128) / 32, l = e % 32;
            sub += ((w[16 + 32 * k + l] >> (2 * j)) & 3) * (int)q8[e];
          }
          isum += (w[g] & 15) * sub;
          summs += (w[g] >> 4) * sext16(ldb16(a + 260 + 2 * g));
        }
        acc += (dy * h2f(ldb16(w + 80))) * (float)isum - (dy * h2f(ldb16(w + 82))) * (float)summs;
      } else if constexpr (iq3(TT)) {
        // grid entries from constant memory; value j of entry e is byte j
        int bsum = 0;
        for (int ib = 0; ib < 8; ++ib) {
          int sumi = 0, ls;
          for (int k = 0; k < 8; ++k) {  // 4-value group k of the sub-block
            uint32_t e, s8;
            if constexpr (TT == TT_IQ3_XXS) {
              const uint32_t aux = (uint32_t)w[66 + 4 * ib] | ((uint32_t)w[67 + 4 * ib] << 8) |
                                   ((uint32_t)w[68 + 4 * ib] << 16) | ((uint32_t)w[69 + 4 * ib] << 24);
              e = kIq3xxsGrid[w[2 + 8 * ib + k]];
              s8 = iq_sign8((aux >> (7 * (k >> 1))) & 127u);
              ls = 2 * (int)(aux >> 28) + 1;
            } else {
              e = kIq3sGrid[w[2 + 8 * ib + k] | (((w[66 + ib] >> k) & 1u) << 8)];
              s8 = w[74 + 4 * ib + (k >> 1)];
              ls = 2 * (int)((w[106 + ib / 2] >> (4 * (ib % 2))) & 15u) + 1;
            }
            for (int j = 0; j < 4; ++j) {
              const int v = (int)((e >> (8 * j)) & 255u);
              const bool neg = (s8 >> (4 * (k & 1) + j)) & 1u;
              sumi += (neg ? -v : v) * (int)q8[32 * ib + 4 * k + j];
            }
          }
          bsum += ls * sumi;
        }
        const float dd = h2f(ldb16(w)) * dy;
        acc += TT == TT_IQ3_XXS ? dd * (float)bsum * 0.25f : dd * (float)bsum;
      } else {  // IQ4_XS
        const float d4d8 = h2f(ldb16(w)) * dy;
        const uint32_t sh = ldb16(w + 2);
        for (int ib = 0; ib < 8; ++ib) {
          const int ls = (int)(((w[4 + ib / 2] >> (4 * (ib % 2))) & 15u) | (((sh >> (2 * ib)) & 3u) << 4));
          int sumi = 0;
          for (int j = 0; j < 32; ++j) {
            const uint32_t q = w[8 + 16 * ib + (j & 15)];
            const uint32_t nib = j < 16 ? (q & 15u) : (q >> 4);
            const uint32_t tab = nib < 4 ? IQ4_T0 : nib < 8 ? IQ4_T1 : nib < 12 ? IQ4_T2 : IQ4_T3;
            sumi += sext8(tab >> (8 * (nib & 3))) * (int)q8[32 * ib + j];
          }
          acc += (d4d8 * (float)(ls - 32)) * (float)sumi;
        }
      }
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

// Tokens per pass: the smallest power of two covering the tokens (at most 8);
// the pass masks the tokens past the end.  Swept on MI355X at the config-5
// shapes: three tokens in one 4-token pass cost 15.8 us against 19.0 us for a
// 2-token and a 1-token pass (Q4_K [17408, 5120]).
int gemv_pick_nt(int tokens) { return tokens > 4 ? 8 : tokens > 2 ? 4 : tokens > 1 ? 2 : 1; }

// the two formats with a K-quant GEMV image (g.kimg)
template <class F>
static hipError_t dispatch_kimg(int ttype, F&& f) {
  if (ttype == TT_Q4_K) return f(std::integral_constant<int, TT_Q4_K>{});
  if (ttype == TT_Q6_K) return f(std::integral_constant<int, TT_Q6_K>{});
  return hipErrorInvalidValue;
}

// One-token grids of fewer than 2048 waves run one wave per workgroup
// rather than four.  Measured on MI355X against four-wave workgroups (GGUF
// rows, pre-quantized, weights rotated): config 1's Q8_0 [6144, 1024] (1536
// waves) 3.84 against 4.30 us, Q8_0 [2048, 2048] (1024) 3.89 against 4.12,
// Q4_K [2560, 2560] (1280) 3.84 against 4.02, Q2_K [9728, 2560] (1622) 5.30
// against 5.41, IQ4_NL [6144, 1024] 3.49 against 3.55; from 2048 waves the
// four-wave workgroups stay ahead (Q4_K [4096, 2560] 4.21 against 4.32,
// Q6_K [4096, 4096] 5.88 against 5.95, Q8_0 [4096, 4096] at 4096 waves 6.10
// against 6.25).  IQ3_XXS / IQ3_S keep four waves: each workgroup first
// copies the format's grid into LDS ([4096, 2560] 5.17 against 5.40).
static constexpr long kGemvOneWaveBelow = 2048;

template <int TT, int NT, int NR, bool IMG = false>
static hipError_t launch_gemv_t(const GemvArgs& g, int team, hipStream_t s) {
  const int upr = g.cols / 64;
  if (team > upr) team = upr;
  if (team > 64) team = 64;
  const int tpw = 64 / team;
  const long teams = (g.rows + NR - 1) / NR;
  const long waves = (teams + tpw - 1) / tpw;
  if constexpr (NT == 1 && !iq3(TT)) {
    if (waves < kGemvOneWaveBelow) {
      hipLaunchKernelGGL((k_gemv<TT, NT, NR, IMG, 1>), dim3((unsigned)waves), dim3(64), 0, s, (const uint8_t*)g.w,
                         (const uint8_t*)g.xq, g.out, g.rows, g.row_bytes, g.act_bytes, upr, team, g.tokens);
      return hipGetLastError();
    }
  }
  const unsigned grid = (unsigned)((waves + 3) / 4);
  hipLaunchKernelGGL((k_gemv<TT, NT, NR, IMG>), dim3(grid), dim3(256), 0, s, (const uint8_t*)g.w,
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
    case 2: return launch_gemv_nr<TT, 2>(g, team, nr, s);
    case 4: return launch_gemv_nr<TT, 4>(g, team, nr, s);
    case 8: return launch_gemv_nr<TT, 8>(g, team, nr, s);
    default: return hipErrorInvalidValue;
  }
}

// Default launch shape for batch-1, from sweeps on MI355X at the benchmark
// shapes.  Long Q6_K / Q4_K rows (>= 8192 / 4096 values) take teams of four /
// two whole waves with two or four rows per team: the activation is shared
// by the rows while the waves in flight stay many (Q6_K [2560, 9728]: 7.6 us
// vs 9.0 us with 64-lane teams; [5120, 17408]: 18.2 vs 21.9 us; Q4_K
// [17408, 5120]: 11.4 vs 12.9 us).  Otherwise Q6_K uses 64 lanes per row,
// Q4_K and IQ4_NL reuse the activation over two or four rows per lane, and
// Q8_0 over two rows when the matrix is large enough to fill the GPU anyway.
// The further formats, swept at [17408, 5120] and [9728, 2560]: Q5_K as Q4_K;
// Q3_K (its decode is VALU-heavy) two-wave teams of four rows on long rows
// (20.5 vs 28.3 us) and 64 lanes per row otherwise; Q2_K and IQ4_XS two rows
// per 20-lane team (10.4 vs 14.2 us, 14.2 vs 17.2 us).  The 4-bit 32-value
// formats, swept at [17408, 5120], [19456, 2560] and [2560, 9728]: four-wave
// teams on rows of >= 8192 values (IQ4_NL 5.8 vs 6.7 us, Q4_0 5.5 vs 6.4,
// Q4_1 5.2 vs 6.4), two-wave teams for Q4_0 / Q4_1 from 4096 values (Q4_1
// 11.5 vs 15.8 us: its 40-byte units need no realignment and stream at
// 4.8 TB/s), else two rows per 40- or 20-lane team.  IQ3_XXS / IQ3_S (grid
// lookups in LDS make their decode VALU-heavy), swept at the same shapes:
// four-wave teams of two rows on rows of >= 8192 values (6.1 vs 7.5 us),
// one row per 20-lane team at width 2560 (9.3 vs 10.1 us), two from 4096.
static void default_shape(const GemvArgs& g, int& team, int& nr) {
  const int upr = g.cols / 64;
  const bool nib32 = g.ttype == TT_Q4_0 || g.ttype == TT_Q4_1 || g.ttype == TT_IQ4_NL;
  // long rows: teams of whole waves (k_gemv_mw), several rows per team (the
  // Q6_K image two: [5120, 17408] 28.2 us with four against 18.1 from the
  // GGUF rows)
  if (g.ttype == TT_Q6_K && upr >= 128) {
    team = 256;
    nr = g.rows >= 4096 && !g.kimg ? 4 : 2;
    return;
  }
  if (nib32 && upr >= 128) {
    team = 256;
    nr = g.ttype == TT_Q4_1 ? 2 : 1;
    return;
  }
  if (iq3(g.ttype) && upr >= 128) {
    team = 256;
    nr = 2;
    return;
  }
  if ((g.ttype == TT_Q4_0 || g.ttype == TT_Q4_1) && upr >= 64) {
    team = 128;
    nr = g.ttype == TT_Q4_1 ? 4 : 2;
    return;
  }
  // Q4_K at width 4096: one-wave teams of two rows ([12288, 4096] 7.56 us
  // against 8.15 with two-wave teams of four)
  if (g.ttype == TT_Q4_K && upr == 64 && g.rows >= 4096) {
    team = 64;
    nr = 2;
    return;
  }
  if ((g.ttype == TT_Q4_K || g.ttype == TT_Q5_K || g.ttype == TT_Q3_K) && upr >= 64) {
    team = 128;
    nr = 4;
    return;
  }
  switch (g.ttype) {
    // Q6_K in 20-lane teams where the units are a multiple of 20 past 64
    // ([17408, 5120] 20.13 us against 22.00 with 64 lanes; at 40 units the
    // 40-lane team stays ahead, [19456, 2560] 12.89 against 14.85)
    case TT_Q6_K: nr = g.rows >= 4096 ? 2 : 1; team = upr > 64 && upr % 20 == 0 ? 20 : 64; break;
    case TT_Q4_K: case TT_Q5_K:
      nr = g.rows >= 16384 && upr <= 40 ? 4 : 2; team = upr <= 40 ? 40 : 20; break;
    case TT_IQ4_NL: nr = 4; team = 20; break;
    case TT_Q4_0: case TT_Q4_1: nr = 2; team = upr <= 40 ? 40 : 20; break;
    case TT_IQ4_XS: case TT_Q2_K: nr = 2; team = 20; break;
    case TT_IQ3_XXS: case TT_IQ3_S: nr = upr >= 64 ? 2 : 1; team = 20; break;
    case TT_Q3_K: nr = 1; team = 64; break;
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

static hipError_t launch_gemv_multiwave(const GemvArgs& g, int nr, int wv, hipStream_t s);

// Balanced teams (k_gemv_bal) for one-token Q6_K matvecs from the K-quant
// image with rows of 64a + b units, 1 <= a <= 4, and >= 4096 rows: one wave
// of two rows where a = 1, four waves of two (a = 3) or four (a = 4) rows
// otherwise.  Measured on MI355X against the default team shapes, weights
// rotated: [5120, 17408] 15.4-15.9 us against 17.4-17.9, [12288, 6144] 12.7
// against 14.9-15.4, [17408, 5120] 15.0 against 17.2, [4096, 12288] 9.2-9.3
// against 9.7-9.8.  Fewer rows keep the default shapes ([2560, 9728] 7.3
// against 6.1: half the waves in flight), and so do the GGUF rows, whose
// misaligned 210-byte super-blocks lose with every load at once ([5120,
// 17408] 21.0 against 19.0 us, [4096, 12288] 12.2 against 11.1).
static bool bal_shape(const GemvArgs& g, int& nr, int& wv) {
  if (!g.kimg || g.ttype != TT_Q6_K || g.tokens != 1 || g.rows < 4096 || g.cols % 256) return false;
  const int upr = g.cols / 64, a = upr / 64, b = upr % 64;
  if (a == 1) {
    nr = 2;
    wv = 1;
  } else if (a == 3 || a == 4) {
    nr = a == 4 ? 4 : 2;
    wv = 4;
  } else {
    return false;
  }
  return nr * b <= 64 * wv;
}

template <int TT, int NR, int WV, bool IMG>
static hipError_t launch_gemv_bal_t(const GemvArgs& g, hipStream_t s) {
  constexpr int TPB = 4 / WV;
  const int upr = g.cols / 64;
  if (upr / 64 < 1 || upr / 64 > WV || NR * (upr % 64) > 64 * WV) return hipErrorInvalidValue;
  const long teams = (g.rows + NR - 1) / NR;
  const unsigned grid = (unsigned)((teams + TPB - 1) / TPB);
  hipLaunchKernelGGL((k_gemv_bal<TT, NR, WV, 1, IMG>), dim3(grid), dim3(256), 0, s, (const uint8_t*)g.w,
                     (const uint8_t*)g.xq, g.out, g.rows, g.row_bytes, upr);
  return hipGetLastError();
}

static hipError_t launch_gemv_bal(const GemvArgs& g, int nr, int wv, hipStream_t s) {
  if (g.ttype != TT_Q6_K || !g.kimg) return hipErrorInvalidValue;
  if (wv == 1 && nr == 2) return launch_gemv_bal_t<TT_Q6_K, 2, 1, true>(g, s);
  if (wv == 4 && nr == 2) return launch_gemv_bal_t<TT_Q6_K, 2, 4, true>(g, s);
  if (wv == 4 && nr == 4) return launch_gemv_bal_t<TT_Q6_K, 4, 4, true>(g, s);
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(const GemvArgs& g, int team, int nt, int nr, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  if (g.kimg && (g.tokens != 1 || !kimage_format(g.ttype) || g.cols % 256)) return hipErrorInvalidValue;
  if (team <= 0 && nr <= 0 && g.tokens == 1) {
    int bwv = 0;
    if (bal_shape(g, nr, bwv)) return launch_gemv_bal(g, nr, bwv, s);
    default_shape(g, team, nr);
  } else if (team <= 0 && nr <= 0 && nt <= 0) {
    // several tokens: each weight unit is decoded once (Prep<TT>) and
    // multiplied by every token of the pass; two rows per lane halve the
    // activation loads per weight load.  Swept on MI355X over 8..64 lanes,
    // 1..4 rows and 2..8 tokens per pass at T = 2..16: Q4_K [17408, 5120]
    // 20 lanes x 2 rows (T = 4: 18.9 us against 22.0 with 16 lanes), four
    // rows from 6 tokens (T = 8: 29.7 vs 31.4 us); Q6_K [5120, 17408] 64
    // lanes x 2 rows; IQ4_NL [17408, 5120] 20 x 2; Q8_0 [3584, 1024] one row
    // (launch-bound either way).
    nr = g.ttype == TT_Q8_0 ? 1 : (g.ttype == TT_Q4_K && g.tokens >= 6) ? 4 : 2;
    team = g.ttype == TT_Q6_K ? 64 : g.ttype == TT_Q8_0 ? 32 : g.ttype == TT_Q4_K || g.ttype == TT_IQ4_NL ? 20 : 16;
  } else {
    if (nr <= 0) nr = 1;
    if (team <= 0) team = gemv_pick_team((g.rows + nr - 1) / nr, g.cols, kGemvTargetWaves);
  }
  if (team > 64) return launch_gemv_multiwave(g, nr, team / 64, s);
  if (nt <= 0) nt = gemv_pick_nt(g.tokens);
  if (g.kimg) {
    return dispatch_kimg(g.ttype, [&](auto tt) -> hipError_t {
      constexpr int T = decltype(tt)::value;
      switch (nr) {
        case 1: return launch_gemv_t<T, 1, 1, true>(g, team, s);
        case 2: return launch_gemv_t<T, 1, 2, true>(g, team, s);
        case 4: return launch_gemv_t<T, 1, 4, true>(g, team, s);
        default: return hipErrorInvalidValue;
      }
    });
  }
  return dispatch_type(g.ttype, [&](auto tt) { return launch_gemv_type<decltype(tt)::value>(g, team, nt, nr, s); });
}

template <int TT, int NR, int WV, bool IMG = false>
static hipError_t launch_gemv_mw_t(const GemvArgs& g, hipStream_t s) {
  constexpr int TPB = 4 / WV;
  const long teams = (g.rows + NR - 1) / NR;
  const unsigned grid = (unsigned)((teams + TPB - 1) / TPB);
  hipLaunchKernelGGL((k_gemv_mw<TT, NR, WV, IMG>), dim3(grid), dim3(256), 0, s, (const uint8_t*)g.w,
                     (const uint8_t*)g.xq, g.out, g.rows, g.row_bytes, g.cols / 64);
  return hipGetLastError();
}

template <int TT, bool IMG = false>
static hipError_t launch_gemv_mw_type(const GemvArgs& g, int nr, int wv, hipStream_t s) {
  if (wv == 2) {
    switch (nr) {
      case 1: return launch_gemv_mw_t<TT, 1, 2, IMG>(g, s);
      case 2: return launch_gemv_mw_t<TT, 2, 2, IMG>(g, s);
      case 4: return launch_gemv_mw_t<TT, 4, 2, IMG>(g, s);
    }
  } else if (wv == 4) {
    switch (nr) {
      case 1: return launch_gemv_mw_t<TT, 1, 4, IMG>(g, s);
      case 2: return launch_gemv_mw_t<TT, 2, 4, IMG>(g, s);
      case 4: return launch_gemv_mw_t<TT, 4, 4, IMG>(g, s);
    }
  }
  return hipErrorInvalidValue;
}

// one token, teams of wv = 2 or 4 waves
static hipError_t launch_gemv_multiwave(const GemvArgs& g, int nr, int wv, hipStream_t s) {
  if (g.tokens != 1) return hipErrorInvalidValue;
  if (g.kimg)
    return dispatch_kimg(g.ttype, [&](auto tt) { return launch_gemv_mw_type<decltype(tt)::value, true>(g, nr, wv, s); });
  return dispatch_type(g.ttype, [&](auto tt) { return launch_gemv_mw_type<decltype(tt)::value>(g, nr, wv, s); });
}

template <int TT, int NR, int WGS>
static hipError_t launch_gemv_q_t(const GemvArgs& g, const float* x, void* xq_out, int team, hipStream_t s) {
  const int upr = g.cols / 64;
  if (team > 64) team = 64;
  const int tpw = 64 / team;
  const long teams = (g.rows + NR - 1) / NR;
  const long waves = (teams + tpw - 1) / tpw;
  const unsigned grid = (unsigned)((waves + WGS / 64 - 1) / (WGS / 64));
  const size_t lds = (size_t)fused_lds_bytes(TT, g.cols);
  hipLaunchKernelGGL((k_gemv_q<TT, NR, WGS>), dim3(grid), dim3(WGS), lds, s, (const uint8_t*)g.w, x,
                     (uint8_t*)xq_out, g.out, g.rows, g.cols, g.row_bytes, upr, team, nullptr, nullptr, 0, 0L);
  return hipGetLastError();
}

template <int TT>
static hipError_t launch_gemv_q_type(const GemvArgs& g, const float* x, void* xq_out, int team, int nr, int wgs,
                                     hipStream_t s) {
  if (wgs == 1024 && nr == 1) return launch_gemv_q_t<TT, 1, 1024>(g, x, xq_out, team, s);
  if (wgs == 1024 && nr == 2) return launch_gemv_q_t<TT, 2, 1024>(g, x, xq_out, team, s);
  if (wgs == 512 && nr == 1) return launch_gemv_q_t<TT, 1, 512>(g, x, xq_out, team, s);
  if (wgs == 512 && nr == 2) return launch_gemv_q_t<TT, 2, 512>(g, x, xq_out, team, s);
  if (wgs != 256) return hipErrorInvalidValue;
  switch (nr) {
    case 1: return launch_gemv_q_t<TT, 1, 256>(g, x, xq_out, team, s);
    case 2: return launch_gemv_q_t<TT, 2, 256>(g, x, xq_out, team, s);
    case 4: return launch_gemv_q_t<TT, 4, 256>(g, x, xq_out, team, s);
    default: return hipErrorInvalidValue;
  }
}

bool gemv_fused_fits(int ttype, int cols) { return fused_lds_bytes(ttype, cols) <= kFusedMaxLds; }

// Default fused shape: one row per lane and 1024-thread workgroups (16 waves
// quantize the activation together, once per workgroup).  Lanes per row: the
// candidate with the fewest wave-steps (waves x units per lane) among those
// whose grid has at least 192 workgroups (three quarters of the CUs), ties to
// the smaller team; if none fills the GPU, the largest grid.  Swept on MI355X
// over Q8_0 [6144, 1024], Q4_K [9728 / 19456, 2560] and [12288, 4096], Q6_K
// [2560, 2560] and IQ4_NL [32768, 2560]: the best shape on five, within 9% on
// the sixth (Q4_K [19456, 2560]: 20 lanes, 8.8 us; 12 lanes 10.0 us).
// Re-swept over 10-64 lanes, 1-2 rows and 256-1024 threads: the tie at
// [12288, 4096] (16, 32 and 64 lanes) goes to 16 lanes (8.97 us; 32 lanes
// 9.56, 64 lanes 10.86); at [19456, 2560] 10 lanes 9.01 against 20 lanes
// 9.10.
static void fused_default_shape(const GemvArgs& g, int& team, int& nr, int& wgs) {
  static const int kCand[] = {8, 10, 16, 20, 32, 40, 64};
  const long upr = g.cols / 64;
  int best = -1;
  long best_w = 0, best_grid = 0;
  bool best_full = false;
  for (int t : kCand) {
    const long tpw = 64 / t;
    const long waves = (g.rows + tpw - 1) / tpw;
    const long grid = (waves + 15) / 16;
    const long w = waves * ((upr + t - 1) / t);
    const bool full = grid >= 192;
    bool take;
    if (best < 0) take = true;
    else if (full != best_full) take = full;
    else if (full) take = w < best_w;           // ties: the earlier (smaller) team
    else take = grid >= best_grid;
    if (take) {
      best = t;
      best_w = w;
      best_grid = grid;
      best_full = full;
    }
  }
  team = best;
  nr = 1;
  wgs = 1024;
}

// Fused quantize + GEMV against separate quantize and GEMV launches, measured
// on MI355X with the default shapes: the fused launch wins for rows up to
// 32768 at widths up to 4096 (Q4_K [19456, 2560] 9.4 vs 10.7 us, Q8_0 [6144,
// 1024] 5.0 vs 6.2 us) and loses on long rows, where every workgroup would
// quantize a long activation (Q6_K [2560, 9728] 12.4 vs 10.4 us, Q4_K
// [17408, 5120] 14.9 vs 14.2 us).  The 32-value formats' separate GEMV takes
// multi-row shapes the fused launch does not, and wins on larger matrices:
// Q8_0 from width 4096 ([12288, 4096] 19.2 vs 22.1 us; [32768, 2560] fused
// 21.0 vs 27.9), the 4-bit ones from 2^24 weights (Q4_0 [19456, 2560] 10.5
// vs 11.9 us, IQ4_NL 11.8 vs 13.7; [6144, 1024] fused 4.7 vs 6.8).
bool gemv_fused_preferred(const GemvArgs& g) {
  if (g.tokens != 1 || !gemv_fused_fits(g.ttype, g.cols) || g.cols > 4096 || g.rows > 32768) return false;
  if (g.ttype == TT_Q8_0) return g.cols <= 2560;
  if (act32(g.ttype)) return (long)g.rows * g.cols <= (1L << 24);
  return true;
}

hipError_t launch_gemv_fused(const GemvArgs& g, const float* x, void* xq_out, int team, int nr, int wgs,
                             hipStream_t s) {
  if (g.rows <= 0) return hipSuccess;
  if (g.tokens != 1 || g.kimg || !gemv_fused_fits(g.ttype, g.cols)) return hipErrorInvalidValue;
  if (team <= 0 && nr <= 0 && wgs <= 0) {
    fused_default_shape(g, team, nr, wgs);
  } else {
    if (nr <= 0) nr = 1;
    if (wgs <= 0) wgs = 256;
    if (team <= 0) team = gemv_pick_team((g.rows + nr - 1) / nr, g.cols, kGemvTargetWaves);
  }
  return dispatch_type(g.ttype, [&](auto tt) {
    return launch_gemv_q_type<decltype(tt)::value>(g, x, xq_out, team, nr, wgs, s);
  });
}

// ---- split-K quantize + GEMV (batch 1, long rows) ---------------------------------
// Workspace: kSkCountBytes of row-tile counters (zero before the first launch,
// zero again after every launch), then the partials [slices][rows] f32.
long gemv_splitk_work_bytes(int rows, int cols) { return kSkCountBytes + 4L * rows * ((cols + 255) / 256); }

__global__ __launch_bounds__(256) void k_fill_zero(uint32_t* __restrict__ p, long n) {
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) p[i] = 0u;
}

hipError_t launch_fill_zero(void* p, long bytes, hipStream_t s) {
  const long n = bytes / 4;
  if (n <= 0) return hipSuccess;
  const long g = (n + 255) / 256;
  hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)(g < 1024 ? g : 1024)), dim3(256), 0, s, (uint32_t*)p, n);
  return hipGetLastError();
}

template <int TT, int NR>
static hipError_t launch_gemv_qsk_t(const GemvArgs& g, const float* x, void* xq_out, int team, int su, void* work,
                                    hipStream_t s) {
  constexpr int WGS = 256;
  const int upr = g.cols / 64;
  const long rpw = (long)(WGS / 64) * (64 / team) * NR;
  const long tiles = (g.rows + rpw - 1) / rpw;
  if (tiles > kSkMaxTiles) return hipErrorInvalidValue;
  const int ns = (upr + su - 1) / su;
  if (ns > 65535) return hipErrorInvalidValue;  // grid y limit
  const long swb = g.row_bytes * su / upr;  // exact: su * 64 values are whole blocks
  const size_t lds = (size_t)fused_lds_bytes(TT, 64 * su);
  unsigned* cnt = (unsigned*)work;
  float* part = (float*)((uint8_t*)work + kSkCountBytes);
  hipLaunchKernelGGL((k_gemv_q<TT, NR, WGS, true>), dim3((unsigned)tiles, (unsigned)ns), dim3(WGS), lds, s,
                     (const uint8_t*)g.w, x, (uint8_t*)xq_out, g.out, g.rows, g.cols, g.row_bytes, upr, team, part,
                     cnt, su, swb);
  return hipGetLastError();
}

// Default split-K shape, from a sweep on MI355X (slices of 256..2048 values,
// 4..32 lanes per row, 1..4 rows per lane) over Q6_K [2560, 9728] and
// [5120, 17408], Q4_K [5120, 17408], and Q5_K, Q3_K, IQ4_XS, Q8_0 at
// [2560, 9728]: eight lanes and one row per lane throughout; slices of 1024
// values (within 0.4 us of the best on every shape), 2048 from width 16384
// (Q4_K [5120, 17408] 14.0 vs 15.9 us).
// Re-swept for Q6_K (1024-4096-value slices, 4-16 lanes, 1-2 rows; two
// runs): [5120, 17408] 4096-value slices of 16 lanes 19.5 / 20.2 us against
// 20.6 / 20.8 with 2048-value slices of 8, [4096, 12288] 2048-value slices
// 14.1 / 14.2 against 14.6 / 14.7; [2560, 9728] and Q4_K [5120, 17408] keep
// the rule above (10.3, 13.4 us).
static void splitk_default_shape(const GemvArgs& g, int& team, int& nr, int& slice) {
  team = 8;
  nr = 1;
  slice = g.cols >= 16384 ? 2048 : 1024;
  if (g.ttype == TT_Q6_K && g.cols >= 16384) {
    slice = 4096;
    team = 16;
  } else if (g.ttype == TT_Q6_K && g.cols >= 12288) {
    slice = 2048;
  }
}

// Split-K against the separate quantize + GEMV launches, same sweep (default
// shape): Q6_K [2560, 9728] 10.3 vs 10.4 us, [5120, 17408] 20.8 vs 21.1;
// Q4_K [5120, 17408] 14.0 vs 17.1; Q5_K 9.7 vs 11.3, Q3_K 9.8 vs 13.8,
// IQ4_XS 9.5 vs 9.7, Q8_0 11.5 vs 13.0 at [2560, 9728].  Rows of >= 8192
// values; narrower rows keep the whole-row fused launch.
bool gemv_splitk_preferred(const GemvArgs& g) {
  return g.tokens == 1 && g.cols >= 8192 && g.cols % 256 == 0 && g.rows <= 65536 &&
         fused_lds_bytes(g.ttype, g.cols >= 16384 ? 2048 : 1024) <= kFusedMaxLds;
}

// The K-quant GEMV image against the GGUF rows, measured on MI355X (weights
// rotated past the Infinity Cache, the same launch shape on both, results
// bit-identical).  Pre-quantized GEMV: Q6_K [2560, 9728] 6.87 vs 7.62 us,
// [19456, 2560] 12.14 vs 12.87, [17408, 5120] 20.71 vs 21.97; Q4_K [17408,
// 5120] 11.52 vs 11.50, [19456, 2560] 8.90 vs 8.15, [12288, 4096] 8.00 vs
// 8.13.  Read by the one-launch quantize + GEMV and its split-K form, the
// image lost (Q4_K [19456, 2560] 9.53 vs 9.38 us, Q6_K [2560, 9728] split
// 10.79 vs 10.20, Q4_K [5120, 17408] split 15.05 vs 14.01), so those keep
// the GGUF rows.  The Exec mirror's batch-1 matvec reads the image for Q6_K
// wherever the whole-row one-launch form is not preferred, quantizing
// separately: Q6_K [17408, 5120] 23.3 vs 26.2 us; and, once k_gemv_mw issued
// every load of a unit before its dots (image GEMV [2560, 9728] 6.05 us,
// [5120, 17408] 16.5), also instead of the split-K form: the config-2 decode
// step (its Q6_K down projection [2560, 9728]) 17.8 against 19.2 us,
// [5120, 17408] 18.4 against 18.3.
bool gemv_kimage_preferred(const GemvArgs& g) {
  return g.tokens == 1 && g.ttype == TT_Q6_K && g.cols % 256 == 0 && !gemv_fused_preferred(g);
}

hipError_t launch_gemv_splitk(const GemvArgs& g, const float* x, void* xq_out, int team, int nr, int slice,
                              void* work, long work_bytes, hipStream_t s) {
  if (g.rows <= 0) return hipSuccess;
  if (g.tokens != 1 || g.kimg || work == nullptr || work_bytes < gemv_splitk_work_bytes(g.rows, g.cols))
    return hipErrorInvalidValue;
  int dt = 0, dn = 0, ds = 0;
  splitk_default_shape(g, dt, dn, ds);
  if (team <= 0) team = dt;
  if (nr <= 0) nr = dn;
  if (slice <= 0) slice = ds;
  if (slice % 256 || (team & (team - 1)) || team < 4 || team > 64) return hipErrorInvalidValue;
  const int su = slice / 64;
  if (fused_lds_bytes(g.ttype, slice) > kFusedMaxLds) return hipErrorInvalidValue;
  return dispatch_type(g.ttype, [&](auto tt) -> hipError_t {
    constexpr int T = decltype(tt)::value;
    switch (nr) {
      case 1: return launch_gemv_qsk_t<T, 1>(g, x, xq_out, team, su, work, s);
      case 2: return launch_gemv_qsk_t<T, 2>(g, x, xq_out, team, su, work, s);
      case 4: return launch_gemv_qsk_t<T, 4>(g, x, xq_out, team, su, work, s);
      default: return hipErrorInvalidValue;
    }
  });
}

hipError_t launch_gemv_generic(const GemvArgs& g, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  const long n = (long)g.rows * g.tokens;
  const unsigned grid = (unsigned)((n + 255) / 256);
  const uint8_t* w = (const uint8_t*)g.w;
  const uint8_t* a = (const uint8_t*)g.xq;
  return dispatch_type(g.ttype, [&](auto tt) {
    hipLaunchKernelGGL(k_gemv_generic<decltype(tt)::value>, dim3(grid), dim3(256), 0, s, w, a, g.out, g.rows,
                       g.cols, g.row_bytes, g.act_bytes, g.tokens);
    return hipGetLastError();
  });
}

template <int TT>
static hipError_t launch_ints_t(const GemvArgs& g, int* ints, hipStream_t s) {
  const int groups = per_block_ints(TT) ? g.cols / 64 : g.cols / 256;
  const long n = (long)g.tokens * g.rows * groups;
  const unsigned grid = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(k_block_ints<TT>, dim3(grid), dim3(256), 0, s, (const uint8_t*)g.w,
                     (const uint8_t*)g.xq, ints, g.rows, groups, g.row_bytes, g.act_bytes, g.tokens);
  return hipGetLastError();
}

hipError_t launch_block_ints(const GemvArgs& g, int* ints, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  return dispatch_type(g.ttype, [&](auto tt) { return launch_ints_t<decltype(tt)::value>(g, ints, s); });
}

}  // namespace qhip
