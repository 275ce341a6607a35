// gemv_image.hip -- batch-1 GEMV of the 32-value formats (IQ4_NL, Q4_0, Q8_0)
// from a GEMV weight image.
//
// Why an image.  An 18-byte block puts its 16 quant bytes at offset 2 of an
// 18-byte stride, so a lane's 16-byte piece of a row is never 16-byte aligned
// and a team's loads touch every cache line of the span more than once; the
// texture path (address processing and tag lookups per line), not HBM, then
// bounds the GEMV (TA busy 76%, TCP 48% of cycles stalled on pending misses
// for IQ4_NL [248320, 2560] at 64% of HBM peak).  The image holds the same
// bytes per row, reordered for the kernel below: a team of T lanes walks a
// row in P passes, lane j taking unit u = pT + j (64 values: blocks 2u and
// 2u+1) in pass p, and every load of a pass is one aligned 16-byte piece per
// lane with the team's lanes contiguous.  T and P depend on the row width
// and, for Q8_0 at one width, the format (img_geom): U = cols / 64 = T P
// units per row.
//
//   row, 36 U bytes (as the GGUF row):
//     [16 ((2p + e) T + j)]        16 quant bytes of block 2u+e (byte i: value
//                                  i in the low nibble, i+16 in the high one)
//     [32 U + 4 (j P + p)]         the f16 scales of blocks 2u (low half) and
//                                  2u+1 (high half): a lane's P pairs adjacent
//   Q8_0 (34-byte blocks: the quants at offset 2 of a 34-byte stride, every
//   16-byte piece misaligned alike), 68 U bytes per row:
//     [16 (((2p + e) 2 + h) T + j)]  quant bytes 16h..16h+15 of block 2u+e
//                                  (the activation's slot order below)
//     [64 U + 4 (j P + p)]         the f16 scales of blocks 2u and 2u+1
//
// The activation is quantized (the same Q8_0 values and scales as the
// reference layout, quantize.hip) into the matching split layout, 72 U bytes
// per token:
//     [16 (((2p + e) 2 + h) T + j)]  values 16h..16h+15 of block 2u+e
//     [64 U + 8 (j P + p)]           the scales of blocks 2u, 2u+1 as f32
//
// Lane j adds its units in pass order and the team folds the lanes with the
// shuffle tree of the GGUF-layout kernel (gemv.hip); each unit's float is
// the same expression, (dw0 da0) s0 + (dw1 da1) s1, with s0 and s1 the
// blocks' exact integer dots.
#include "qhip_device.hpp"
#include "qhip_internal.hpp"

namespace qhip {

bool gemv_image_format(int ttype) { return ttype == TT_IQ4_NL || ttype == TT_Q4_0 || ttype == TT_Q8_0; }

// 16-byte quant slots per 32-value block: the 4-bit formats one, Q8_0 two
template <int TT>
__host__ __device__ constexpr int img_qs() { return TT == TT_Q8_0 ? 2 : 1; }

// Team width and passes for a row width.  Swept on MI355X over T = 8..64 and
// one, two or four rows per team: 20-lane teams wherever U is a multiple of
// 20 (IQ4_NL [248320, 2560] 61.3 us, 8-lane 67.1, 10-lane 67.5), whole-wave
// teams at width 4096 (5.5 us, 32-lane 5.8, 16-lane 6.1); 32- and 16-lane
// teams otherwise.  At width 5120 IQ4_NL takes 16-lane teams of five passes,
// every lane of the wave busy ([17408, 5120] 11.93 us against 12.58 with 20
// lanes x 4 passes, 13.4 with 40 x 2, in a standalone harness; 12.07-12.38
// against 12.48-12.55 through the C ABI), while Q4_0, whose decode is
// lighter, keeps 20 lanes (11.5-11.7 against 11.7-12.0 with 16); Q8_0 (two
// 16-byte slots per block, twice the quant bytes per unit) takes 40-lane
// teams of two passes: 17.8 us against 18.9 with 20 lanes and 19.6 with 16.
static bool img_geom(int ttype, int cols, int& T, int& P) {
  if (cols <= 0 || cols % 64) return false;
  const int U = cols / 64;
  if (ttype == TT_Q8_0 && U == 80) { T = 40; P = 2; return true; }
  if (ttype == TT_IQ4_NL && U == 80) { T = 16; P = 5; return true; }
  if (U % 20 == 0 && U / 20 <= 4) { T = 20; P = U / 20; return true; }
  if (U % 64 == 0 && U / 64 <= 2) { T = 64; P = U / 64; return true; }
  if (U % 32 == 0 && U / 32 <= 4) { T = 32; P = U / 32; return true; }
  if (U % 16 == 0 && U / 16 <= 4) { T = 16; P = U / 16; return true; }
  return false;
}

bool gemv_image_width(int cols) {
  int T, P;
  return img_geom(TT_IQ4_NL, cols, T, P);
}

int gemv_image_layout(int ttype, int cols) {
  int T, P;
  return img_geom(ttype, cols, T, P) ? 16 * T + P : -1;
}

// One block's integer dot (kernels32.c:342-361, :447-464): the quant slots q
// (4-bit: one, both halves; Q8_0: two, values 0..15 and 16..31) against
// activation values 0..15 (y0) and 16..31 (y1).
template <int TT>
__device__ __forceinline__ int img_block(const u32x4 (&q)[img_qs<TT>()], const u32x4& y0, const u32x4& y1) {
  const uint32_t qq[4] = {q[0].x, q[0].y, q[0].z, q[0].w};
  const uint32_t ya[4] = {y0.x, y0.y, y0.z, y0.w};
  const uint32_t yb[4] = {y1.x, y1.y, y1.z, y1.w};
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (TT == TT_IQ4_NL) {
      s = iq4_dot8(qq[i], ya[i], yb[i], s);
    } else if constexpr (TT == TT_Q4_0) {
      s = dot4(nib_minus8(qq[i] & 0x0F0F0F0Fu), ya[i], s);
      s = dot4(nib_minus8((qq[i] >> 4) & 0x0F0F0F0Fu), yb[i], s);
    } else {
      const uint32_t q1[4] = {q[img_qs<TT>() - 1].x, q[img_qs<TT>() - 1].y, q[img_qs<TT>() - 1].z,
                              q[img_qs<TT>() - 1].w};
      s = dot4(qq[i], ya[i], s);
      s = dot4(q1[i], yb[i], s);
    }
  }
  return s;
}

// A team of T lanes owns NR consecutive rows (64 / T teams per wave).  The
// passes are unrolled, so the compiler issues a pass's loads ahead of the
// previous pass's arithmetic.  The activation is read from an LDS copy made
// once per workgroup.
template <int TT, int T, int P, int NR>
__global__ __launch_bounds__(256) void k_gemv_img(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XA,
                                                   float* __restrict__ Y, int rows, long row_bytes) {
  constexpr int U = T * P, TPW = 64 / T, QS = img_qs<TT>();
  const int lane = threadIdx.x & 63;
  const int r = lane / T, j = lane - r * T;
  const long row0 = (((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * TPW + r) * NR;
  const bool active = r < TPW && row0 < rows;
  // 4-bit types at two rows per team load before the barrier on every lane
  // (below); the lanes past the wave's teams then address its last team's
  // rows (their loads repeat pieces of the same instruction: no extra
  // traffic)
  constexpr bool EARLY = QS == 1 && NR == 2;
  const long rowa = !EARLY || r < TPW ? row0 : row0 - (long)(r - TPW + 1) * NR;
  float acc[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) acc[k] = 0.0f;
  // the split activation (72 U bytes) once per workgroup into LDS: its
  // 16-byte pieces are read by every team of the workgroup, so through the
  // texture path they cost as much as the weights (IQ4_NL [248320, 2560]
  // 58.5 against 59.1 us, [32768, 2560] 11.0 against 11.4; Q8_0 [17408,
  // 5120] 17.2 against 18.4; the same bits)
  __shared__ __attribute__((aligned(16))) uint8_t xs[72 * U];
  // EARLY: every weight load of the lane is issued before the activation
  // copy (unconditionally: a lane past the teams or the rows reads a valid
  // row and discards it), so that all of a wave's pieces are in flight at
  // once from the start (IQ4_NL [248320, 2560] 58.4 against 58.8-59.6 us,
  // [32768, 2560] 10.9 against 11.3, the same bits).  One row per team
  // ([17408, 5120] 16 x 5: 11.9 against 12.9 us) and Q8_0, with twice the
  // pieces, load pass by pass after the barrier (Q8_0 in 40-lane teams:
  // 17.1 against 17.6-17.7 us at [17408, 5120] all loads first, but 5.9
  // against 5.75 at [4096, 5120]).
  const uint8_t* wr[NR];
#pragma unroll
  for (int k = 0; k < NR; ++k) wr[k] = W + (rowa + k < rows ? rowa + k : rows - 1) * row_bytes;
  uint32_t ws[NR][P];
  u32x4 qa[EARLY ? P : 1][NR][2][QS];
  auto load_ws = [&]() {
#pragma unroll
    for (int k = 0; k < NR; ++k)
#pragma unroll
      for (int p = 0; p < P; ++p) ws[k][p] = ld32(wr[k] + 32 * QS * U + 4 * (j * P + p));
  };
  auto load_pass = [&](int p, u32x4 (&q)[NR][2][QS]) {
#pragma unroll
    for (int k = 0; k < NR; ++k)
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int h = 0; h < QS; ++h) q[k][e][h] = ld128(wr[k] + (((2 * p + e) * QS + h) * T + j) * 16);
  };
  if constexpr (EARLY) {
    load_ws();
#pragma unroll
    for (int p = 0; p < P; ++p) load_pass(p, qa[p]);
  }
  for (int i = threadIdx.x; i < 72 * U / 16; i += 256) *(u32x4*)(xs + 16 * i) = ld128(XA + 16 * i);
  __syncthreads();
  if (active) {
    if constexpr (!EARLY) load_ws();
    float2 ad[P];
#pragma unroll
    for (int p = 0; p < P; ++p) ad[p] = *(const float2*)(xs + 64 * U + 8 * (j * P + p));
#pragma unroll
    for (int p = 0; p < P; ++p) {
      u32x4 q[NR][2][QS];
      if constexpr (EARLY) {
#pragma unroll
        for (int k = 0; k < NR; ++k)
#pragma unroll
          for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int h = 0; h < QS; ++h) q[k][e][h] = qa[p][k][e][h];
      } else {
        load_pass(p, q);
      }
      u32x4 y[2][2];
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int h = 0; h < 2; ++h) y[e][h] = *(const u32x4*)(xs + (((2 * p + e) * 2 + h) * T + j) * 16);
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const int s0 = img_block<TT>(q[k][0], y[0][0], y[0][1]);
        const int s1 = img_block<TT>(q[k][1], y[1][0], y[1][1]);
        acc[k] += (h2f(ws[k][p] & 0xFFFFu) * ad[p].x) * (float)s0 + (h2f(ws[k][p] >> 16) * ad[p].y) * (float)s1;
      }
    }
  }
  // segmented tree over the team (the order depends only on T)
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    if (off < T) {
#pragma unroll
      for (int k = 0; k < NR; ++k) {
        const float v = __shfl_down(acc[k], off, 64);
        if (j + off < T) acc[k] += v;
      }
    }
  }
  if (active && j == 0) {
#pragma unroll
    for (int k = 0; k < NR; ++k)
      if (row0 + k < rows) Y[row0 + k] = acc[k];
  }
}

// GGUF rows -> image rows; one thread per (row, unit).
__global__ __launch_bounds__(256) void k_gemv_img_prepare(const uint8_t* __restrict__ W, uint8_t* __restrict__ img,
                                                           long units, int T, int P, long row_bytes, int q8) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= units) return;
  const int U = T * P;
  const long row = i / U;
  const int u = (int)(i - row * U), p = u / T, j = u - p * T;
  if (q8) {
    // Q8_0: the unit's 68 bytes (two blocks), dword aligned; block 0: d =
    // bytes 0..1, quants 2..33; block 1: d = bytes 34..35, quants 36..67
    const uint8_t* src = W + row * row_bytes + 68L * u;
    uint8_t* dst = img + row * row_bytes;
    uint32_t v[17];
#pragma unroll
    for (int k = 0; k < 17; ++k) v[k] = ld32(src + 4 * k);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const u32x4 qe = {funnel(v[4 * h + 1], v[4 * h], 2), funnel(v[4 * h + 2], v[4 * h + 1], 2),
                        funnel(v[4 * h + 3], v[4 * h + 2], 2), funnel(v[4 * h + 4], v[4 * h + 3], 2)};
      const u32x4 qo = {v[9 + 4 * h], v[10 + 4 * h], v[11 + 4 * h], v[12 + 4 * h]};
      *(u32x4*)(dst + 16L * (((2 * p) * 2 + h) * T + j)) = qe;
      *(u32x4*)(dst + 16L * (((2 * p + 1) * 2 + h) * T + j)) = qo;
    }
    *(uint32_t*)(dst + 64L * U + 4L * (j * P + p)) = (v[0] & 0xFFFFu) | (v[8] & 0xFFFF0000u);
    return;
  }
  const uint8_t* src = W + row * row_bytes + 36L * u;
  uint8_t* dst = img + row * row_bytes;
  uint32_t v[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) v[k] = ld32(src + 4 * k);  // the unit's 36 bytes, dword aligned
  // even block: d = bytes 0..1, quants = bytes 2..17; odd block: d = bytes
  // 18..19, quants = bytes 20..35
  const u32x4 qe = {funnel(v[1], v[0], 2), funnel(v[2], v[1], 2), funnel(v[3], v[2], 2), funnel(v[4], v[3], 2)};
  const u32x4 qo = {v[5], v[6], v[7], v[8]};
  *(u32x4*)(dst + 16L * ((2 * p) * T + j)) = qe;
  *(u32x4*)(dst + 16L * ((2 * p + 1) * T + j)) = qo;
  *(uint32_t*)(dst + 32L * U + 4L * (j * P + p)) = (v[0] & 0xFFFFu) | (v[4] & 0xFFFF0000u);
}

// f32 -> split Q8_0 activation; one thread per value, 32 per block (the
// values and scales of k_quantize_q8_0).
__global__ __launch_bounds__(256) void k_quantize_q8_0_img(const float* __restrict__ x, uint8_t* __restrict__ out,
                                                            long nblocks, int T, int P, long x_stride) {
  const long b = ((long)blockIdx.x * 256 + threadIdx.x) >> 5;
  const int i = threadIdx.x & 31;
  const long t = blockIdx.y;
  const bool ok = b < nblocks;
  const float v = ok ? x[t * x_stride + 32 * b + i] : 0.0f;
  uint32_t hb;
  const int q = quant_q8_0_lane(v, hb);
  if (ok) {
    const int U = T * P;
    uint8_t* o = out + t * 72L * U;
    const int u = (int)(b >> 1), e = (int)(b & 1), h = i >> 4;
    const int p = u / T, j = u - p * T;
    o[16L * (((2 * p + e) * 2 + h) * T + j) + (i & 15)] = (uint8_t)(int8_t)q;
    if (i == 0) *(float*)(o + 64L * U + 8L * (j * P + p) + 4 * e) = h2f(hb);
  }
}

long gemv_image_act_bytes(int cols, int tokens) { return 72L * (cols / 64) * tokens; }

hipError_t launch_gemv_image_prepare(const void* w, long row_bytes, int rows, int cols, void* img, hipStream_t s,
                                     int ttype) {
  int T, P;
  if (!img_geom(ttype, cols, T, P)) return hipErrorInvalidValue;
  const bool q8 = ttype == TT_Q8_0;
  const long units = (long)rows * (T * P);
  if (units <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_gemv_img_prepare, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, s,
                     (const uint8_t*)w, (uint8_t*)img, units, T, P, row_bytes, q8 ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_quantize_act_image(int ttype, const float* x, void* out, int cols, int tokens, long x_stride,
                                     hipStream_t s) {
  int T, P;
  if (!img_geom(ttype, cols, T, P)) return hipErrorInvalidValue;
  const long nblocks = cols / 32;
  if (tokens <= 0) return hipSuccess;
  dim3 grid((unsigned)((nblocks * 32 + 255) / 256), (unsigned)tokens);
  hipLaunchKernelGGL(k_quantize_q8_0_img, grid, dim3(256), 0, s, x, (uint8_t*)out, nblocks, T, P, x_stride);
  return hipGetLastError();
}

template <int TT, int T, int P, int NR>
static hipError_t launch_img_t(const GemvArgs& g, hipStream_t s) {
  constexpr int TPW = 64 / T;
  const long teams = (g.rows + NR - 1) / NR;
  const long waves = (teams + TPW - 1) / TPW;
  const unsigned grid = (unsigned)((waves + 3) / 4);
  hipLaunchKernelGGL((k_gemv_img<TT, T, P, NR>), dim3(grid), dim3(256), 0, s, (const uint8_t*)g.w,
                     (const uint8_t*)g.xq, g.out, g.rows, g.row_bytes);
  return hipGetLastError();
}

template <int TT, int T, int P>
static hipError_t launch_img_nr(const GemvArgs& g, int nr, hipStream_t s) {
  return nr == 2 ? launch_img_t<TT, T, P, 2>(g, s) : launch_img_t<TT, T, P, 1>(g, s);
}

template <int TT>
static hipError_t launch_img_tt(const GemvArgs& g, int T, int P, int nr, hipStream_t s) {
#define QHIP_IMG(TV, PV) \
  if (T == TV && P == PV) return launch_img_nr<TT, TV, PV>(g, nr, s);
  QHIP_IMG(20, 1) QHIP_IMG(20, 2) QHIP_IMG(20, 3) QHIP_IMG(20, 4)
  QHIP_IMG(64, 1) QHIP_IMG(64, 2)
  QHIP_IMG(32, 1) QHIP_IMG(32, 2) QHIP_IMG(32, 3) QHIP_IMG(32, 4)
  QHIP_IMG(16, 1) QHIP_IMG(16, 2) QHIP_IMG(16, 3) QHIP_IMG(16, 4) QHIP_IMG(16, 5)
  if constexpr (TT == TT_Q8_0) {
    QHIP_IMG(40, 2)
  }
#undef QHIP_IMG
  return hipErrorInvalidValue;
}

// Quantize + image GEMV against the GGUF-layout launches (one token),
// measured on MI355X (IQ4_NL, weights rotated past the Infinity Cache; GEMV
// alone, then quantize + GEMV against the one-launch fused form): [248320,
// 2560] 62.8 vs 72.6 us, 64.9 vs 74.7 (fused 79.1); [17408, 5120] 12.2 vs
// 15.3; [19456, 2560] 8.2 vs 9.4, 10.6 vs 11.9 (fused 13.2); [8192, 4096]
// 5.5 vs 7.0; [4096, 4096] 4.0 vs 4.8, 7.5 vs 7.8 (fused 8.1); [12288,
// 2048] 4.8 vs 7.6; Q4_0 alike.  Below 2^23 weights the fused launch wins
// ([6144, 1024]: fused 5.1 us, quantize + image GEMV 7.2).
bool gemv_image_preferred(const GemvArgs& g) {
  return g.tokens == 1 && gemv_image_format(g.ttype) && gemv_image_width(g.cols) &&
         (long)g.rows * g.cols > (1L << 23);
}

// ---- K-quant GEMV image (Q4_K, Q6_K) --------------------------------------------
// The layout is KImg's (qhip_device.hpp): the GGUF row's bytes with each
// unit's 16-byte pieces grouped by piece over chunks of 64 units, so that the
// lanes of a wave, taking consecutive units, load one contiguous span per
// instruction; the headers (Q4_K) or scales and d (Q6_K) after the pieces.
// The GEMV, fused and split-K launchers of gemv.hip read it when g.kimg, with
// the activation in the reference Q8_K layout.
bool gemv_kimage_format(int ttype) { return kimage_format(ttype); }

// GGUF rows -> K-quant image rows; one thread per (row, unit).  The GGUF
// bytes are read 4-byte (Q4_K) or 2-byte (Q6_K: 210-byte super-blocks)
// aligned; Q4_K image rows are 16-byte aligned (144 bytes per super-block),
// Q6_K ones 2-byte aligned and written in 2-byte pieces.
template <int TT>
__global__ __launch_bounds__(256) void k_kimg_prepare(const uint8_t* __restrict__ W, uint8_t* __restrict__ img,
                                                       long units, int U, long row_bytes) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= units) return;
  const long row = i / U;
  const int u = (int)(i - row * U), c = u >> 6, ii = u & 63, m = min(64, U - (c << 6));
  const uint8_t* src = W + row * row_bytes;
  uint8_t* dst = img + row * row_bytes;
  if constexpr (TT == TT_Q4_K) {
    const uint8_t* blk = src + 144L * (u >> 2);
    const int q = u & 3;
    const u32x4 a = {ld32(blk + 16 + 32 * q), ld32(blk + 20 + 32 * q), ld32(blk + 24 + 32 * q), ld32(blk + 28 + 32 * q)};
    const u32x4 b = {ld32(blk + 32 + 32 * q), ld32(blk + 36 + 32 * q), ld32(blk + 40 + 32 * q), ld32(blk + 44 + 32 * q)};
    *(u32x4*)(dst + 16L * (128 * c + ii)) = a;
    *(u32x4*)(dst + 16L * (128 * c + m + ii)) = b;
    if (q == 0) *(u32x4*)(dst + 32L * U + 16 * (u >> 2)) = u32x4{ld32(blk), ld32(blk + 4), ld32(blk + 8), ld32(blk + 12)};
  } else {
    const uint8_t* blk = src + 210L * (u >> 2);
    const int h = (u >> 1) & 1, lh = u & 1;
    auto cp16 = [](const uint8_t* from, uint8_t* to) {
#pragma unroll
      for (int k = 0; k < 8; ++k) ((uint16_t*)to)[k] = ((const uint16_t*)from)[k];
    };
    cp16(blk + 64 * h + 16 * lh, dst + 16L * (192 * c + ii));
    cp16(blk + 64 * h + 32 + 16 * lh, dst + 16L * (192 * c + m + ii));
    cp16(blk + 128 + 32 * h + 16 * lh, dst + 16L * (192 * c + 2 * m + ii));
    const uint8_t* sc = blk + 192 + 8 * h + lh;  // sc[8h + lh + 2q] for q = 0..3
    uint16_t* so = (uint16_t*)(dst + 48L * U + 4 * u);
    so[0] = (uint16_t)(sc[0] | (sc[2] << 8));
    so[1] = (uint16_t)(sc[4] | (sc[6] << 8));
    if ((u & 3) == 0) *(uint16_t*)(dst + 52L * U + 2 * (u >> 2)) = *(const uint16_t*)(blk + 208);
  }
}

hipError_t launch_kimage_prepare(int ttype, const void* w, long row_bytes, int rows, int cols, void* img,
                                 hipStream_t s) {
  if (!kimage_format(ttype) || cols <= 0 || cols % 256) return hipErrorInvalidValue;
  const int U = cols / 64;
  const long units = (long)rows * U;
  if (units <= 0) return hipSuccess;
  const dim3 grid((unsigned)((units + 255) / 256));
  if (ttype == TT_Q4_K)
    hipLaunchKernelGGL(k_kimg_prepare<TT_Q4_K>, grid, dim3(256), 0, s, (const uint8_t*)w, (uint8_t*)img, units, U,
                       row_bytes);
  else
    hipLaunchKernelGGL(k_kimg_prepare<TT_Q6_K>, grid, dim3(256), 0, s, (const uint8_t*)w, (uint8_t*)img, units, U,
                       row_bytes);
  return hipGetLastError();
}

// g.w = the image, g.xq = the split activation of one token.  nr: rows per
// team, 1 or 2 (0 = two rows from 65536 rows: IQ4_NL [248320, 2560] 62.7 vs
// 65.9 us one row; [32768, 2560] 11.4 vs 11.6 us two rows, [17408, 5120]
// 12.2 vs 12.9).
hipError_t launch_gemv_image(const GemvArgs& g, int nr, hipStream_t s) {
  if (g.rows <= 0) return hipSuccess;
  int T, P;
  if (g.tokens != 1 || !gemv_image_format(g.ttype) || !img_geom(g.ttype, g.cols, T, P)) return hipErrorInvalidValue;
  if (nr <= 0) nr = g.rows >= 65536 ? 2 : 1;
  if (nr > 2) return hipErrorInvalidValue;
  if (g.ttype == TT_IQ4_NL) return launch_img_tt<TT_IQ4_NL>(g, T, P, nr, s);
  if (g.ttype == TT_Q8_0) return launch_img_tt<TT_Q8_0>(g, T, P, nr, s);
  return launch_img_tt<TT_Q4_0>(g, T, P, nr, s);
}

}  // namespace qhip
