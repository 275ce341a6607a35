// mmq.hip -- batched / ragged quantized matrix product (prefill) on int8 MFMA.
//
// out[t*rows + r] = W[r] . xq[t] for many tokens at once (reference contract:
// src/kernels/cuda/mmq.cu:2232-2336, reached from mmvq.cu:789 when tokens > 1).
//
// Tiling.  A workgroup of four waves owns a BT-token x BR-row output tile; the
// waves split it 2 x 2 and each wave covers its quarter with 32x32 MFMA
// tiles.  The K dimension is walked in chunks of 256 values: the chunk's
// weight bytes (BR rows) and activation bytes (BT tokens) are decoded into
// plain int8 rows in LDS (IQ4_NL codebook lookup, Q4_K nibbles, Q6_K 6-bit
// values minus 32), plus each format's scales, then the MFMAs read aligned
// 16-byte fragments from there.
//
// Operand roles.  MFMA operand A carries the activations (tile rows = tokens),
// operand B the weights (tile columns = rows), so in the accumulator layout
// every lane holds ONE weight row and 16 tokens: weight-side scales are lane
// scalars, token-side scales are read per element.
//
// Exactness.  Each MFMA covers exactly one scale group of the format, so its
// int32 result is the reference's per-block integer:
//   Q8_0, IQ4_NL  v_mfma_i32_32x32x32_i8 per 32-value block
//                 (src/kernels/x86/kernels32.c:447-464, :342-361)
//   Q4_0, Q4_1    the same on nib - 8 (Q4_0) or the unsigned nibble (Q4_1,
//                 whose min term m * dy * sumy is a rank-1 update in the
//                 epilogue)  (kernels32.c:297-340)
//   Q4_K          v_mfma_i32_32x32x32_i8 per 32-value sub-block on the
//                 nibbles times the two halves of its 6-bit scale (sc = 8 sh
//                 + sl, each product <= 105 fits int8), accumulated over the
//                 super-block in two chains, isum = 8 C_hi + C_lo; the mins term
//                 sum_j bsum[j]*min[j/2] as an exact f16 MFMA (K = 16
//                 bsums, all partial sums < 2^24)  (kernels256.c:474-498)
//   Q6_K          v_mfma_i32_32x32x16_i8 per 16-value group, times its int8
//                 scale in integer arithmetic  (kernels256.c:720-738)
//   Q5_K          as Q4_K on the 5-bit values  (kernels256.c:605-629)
//   IQ4_XS        as Q4_K on the codebook values with the signed scale
//                 ls - 32, no mins  (iq_kernels.c:967-1001)
//   IQ3_XXS/IQ3_S the same on the signed grid values with the odd scale
//                 2 ls + 1  (iq_kernels.c:612-643, :1728-1772)
//   Q3_K          as Q6_K on q3 in [-4, 3] with the signed 6-bit group
//                 scales sc - 32  (kernels256.c:349-369)
//   Q2_K          as Q6_K on q2 in [0, 3] with the 4-bit group scales; the
//                 mins term sum_g bsum[g]*min[g] as Q4_K's f16 MFMA
//                 (kernels256.c:232-257)
// and the float scaling follows per block / super-block.  For the 32-value
// formats the accumulator input is the bit pattern of 1.5*2^23, so the MFMA
// result read as a float is 1.5*2^23 + sumi exactly (|sumi| <= 2^19); one
// fma removes the offset while applying the weight scale:
//   dw*sumi = fma(F, dw, -1.5*2^23*dw)      (the product -1.5*2^23*dw is exact)
// which saves the int->float conversion per element.
#include "qhip_device.hpp"
#include "qhip_internal.hpp"

#include <type_traits>

namespace qhip {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef long i64x1_a8 __attribute__((aligned(8)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

constexpr int kChunk = 256;         // values per staged K-chunk
constexpr int kQS = kChunk + 16;    // LDS bytes per int8 row (pad: rows 4 banks apart)
constexpr float kBias = 12582912.0f;  // 1.5 * 2^23
constexpr int kBiasBits = 0x4B400000;

// ---- LDS images ---------------------------------------------------------------------
template <int TT, int BT, int BR, bool K32 = act32(TT)>
struct MmqSmem;

template <int TT, int BT, int BR>
struct alignas(16) MmqSmem<TT, BT, BR, true> {
  uint8_t aq[BT * kQS];
  uint8_t bq[BR * kQS];
  float ad[8][BT];  // activation block scales of the chunk
  float wd[8][BR];  // weight block scales
};

// Q4_1 adds the block mins: ay = dy * (sum of the activation block's int8s),
// wm = m, so a block contributes wm[r] * ay[t] beside its integer product.
template <int BT, int BR>
struct alignas(16) MmqSmem<TT_Q4_1, BT, BR, true> {
  uint8_t aq[BT * kQS];
  uint8_t bq[BR * kQS];
  float ad[8][BT];
  float wd[8][BR];
  float ay[8][BT];
  float wm[8][BR];
};

template <int BT, int BR>
struct alignas(16) MmqSmem<TT_Q4_K, BT, BR, false> {
  uint8_t aq[BT * kQS];
  uint8_t bq[BR * kQS];
  _Float16 abs[BT][16];  // activation 16-value sums (exact in f16: |bsum| <= 2032)
  _Float16 wmn[BR][16];  // min of the sub-block of each 16-value group
  float ady[BT];
  float wd[BR], wdmin[BR];
  uint32_t wsc[BR][2];  // eight 6-bit sub-block scales, one per byte
};

// Q5_K shares Q4_K's scales and mins; IQ4_XS uses the same per-sub-block
// integer scale bytes (ls - 32, signed) and d, without mins.
template <int BT, int BR>
struct alignas(16) MmqSmem<TT_Q5_K, BT, BR, false> : MmqSmem<TT_Q4_K, BT, BR, false> {};
template <int BT, int BR>
struct alignas(16) MmqSmem<TT_IQ4_XS, BT, BR, false> : MmqSmem<TT_Q4_K, BT, BR, false> {};
// the IQ3 formats: the same image with the odd sub-block scale 2 ls + 1
template <int BT, int BR>
struct alignas(16) MmqSmem<TT_IQ3_XXS, BT, BR, false> : MmqSmem<TT_Q4_K, BT, BR, false> {};
template <int BT, int BR>
struct alignas(16) MmqSmem<TT_IQ3_S, BT, BR, false> : MmqSmem<TT_Q4_K, BT, BR, false> {};

template <int BT, int BR>
struct alignas(16) MmqSmem<TT_Q6_K, BT, BR, false> {
  uint8_t aq[BT * kQS];
  uint8_t bq[BR * kQS];
  float ady[BT];
  float wd[BR];
  uint32_t wsc[BR][4];  // sixteen int8 group scales
};

// Q3_K: sixteen signed group scales (sc - 32) and d, like Q6_K
template <int BT, int BR>
struct alignas(16) MmqSmem<TT_Q3_K, BT, BR, false> : MmqSmem<TT_Q6_K, BT, BR, false> {};

// Q2_K: sixteen 4-bit group scales and mins, d and dmin; the mins term is the
// f16 MFMA of Q4_K over the activation's 16-value sums
template <int BT, int BR>
struct alignas(16) MmqSmem<TT_Q2_K, BT, BR, false> {
  uint8_t aq[BT * kQS];
  uint8_t bq[BR * kQS];
  _Float16 abs[BT][16];
  _Float16 wmn[BR][16];
  uint32_t wsc[BR][4];
  float ady[BT];
  float wd[BR], wdmin[BR];
};

__device__ __forceinline__ void st16(uint8_t* p, uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  *(uint4*)p = make_uint4(a, b, c, d);
}

// q6 - 32 on four packed 6-bit values: flip bit 5, then sign-extend from it
__device__ __forceinline__ uint32_t q6_minus32(uint32_t v) {
  const uint32_t x = v ^ 0x20202020u;
  const uint32_t s = x & 0x20202020u;
  return x | (s << 1) | (s << 2);
}

__device__ __forceinline__ uint32_t f16_pair(uint32_t n) {
  const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)(float)n);
  return h | (h << 16);
}

__device__ __forceinline__ int sext24(int v) { return (v << 8) >> 8; }

// ---- staging: weights ---------------------------------------------------------------
// Staging is split in two so that the global loads of chunk c+1 are in flight
// while chunk c is multiplied: the Unit<> loaders fill registers, emit_w /
// emit_a decode those registers into the LDS image after the barrier.
//
// emit_w: weight unit u4 (0..3) of the chunk, local row `row`
template <int TT, int BT, int BR>
__device__ __forceinline__ void emit_w(MmqSmem<TT, BT, BR>& sm, const typename Unit<TT>::W& w, int row,
                                       int u4) {
  uint8_t* dst = sm.bq + row * kQS + 64 * u4;
  if constexpr (TT == TT_Q8_0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) st16(dst + 16 * i, w.q[4 * i], w.q[4 * i + 1], w.q[4 * i + 2], w.q[4 * i + 3]);
    sm.wd[2 * u4][row] = h2f(w.d0);
    sm.wd[2 * u4 + 1][row] = h2f(w.d1);
  } else if constexpr (TT == TT_IQ4_NL) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint32_t* q = w.q + 4 * b;
      st16(dst + 32 * b, iq4_lo(q[0]), iq4_lo(q[1]), iq4_lo(q[2]), iq4_lo(q[3]));
      st16(dst + 32 * b + 16, iq4_hi(q[0]), iq4_hi(q[1]), iq4_hi(q[2]), iq4_hi(q[3]));
    }
    sm.wd[2 * u4][row] = h2f(w.d0);
    sm.wd[2 * u4 + 1][row] = h2f(w.d1);
  } else if constexpr (TT == TT_Q4_0 || TT == TT_Q4_1) {
    // Q4_0: nib - 8; Q4_1: the unsigned nibble (its min is added apart)
    const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint32_t* q = w.q + 4 * b;
      if constexpr (TT == TT_Q4_0) {
        st16(dst + 32 * b, nib_minus8(q[0] & m), nib_minus8(q[1] & m), nib_minus8(q[2] & m), nib_minus8(q[3] & m));
        st16(dst + 32 * b + 16, nib_minus8((q[0] >> 4) & m), nib_minus8((q[1] >> 4) & m),
             nib_minus8((q[2] >> 4) & m), nib_minus8((q[3] >> 4) & m));
      } else {
        st16(dst + 32 * b, q[0] & m, q[1] & m, q[2] & m, q[3] & m);
        st16(dst + 32 * b + 16, (q[0] >> 4) & m, (q[1] >> 4) & m, (q[2] >> 4) & m, (q[3] >> 4) & m);
      }
    }
    if constexpr (TT == TT_Q4_0) {
      sm.wd[2 * u4][row] = h2f(w.d0);
      sm.wd[2 * u4 + 1][row] = h2f(w.d1);
    } else {
      sm.wd[2 * u4][row] = h2f(w.h0);
      sm.wd[2 * u4 + 1][row] = h2f(w.h1);
      sm.wm[2 * u4][row] = h2f(w.h0 >> 16);
      sm.wm[2 * u4 + 1][row] = h2f(w.h1 >> 16);
    }
  } else if constexpr (TT == TT_Q4_K) {
    const uint32_t m = 0x0F0F0F0Fu;
    st16(dst, w.q[0] & m, w.q[1] & m, w.q[2] & m, w.q[3] & m);
    st16(dst + 16, w.q[4] & m, w.q[5] & m, w.q[6] & m, w.q[7] & m);
    st16(dst + 32, (w.q[0] >> 4) & m, (w.q[1] >> 4) & m, (w.q[2] >> 4) & m, (w.q[3] >> 4) & m);
    st16(dst + 48, (w.q[4] >> 4) & m, (w.q[5] >> 4) & m, (w.q[6] >> 4) & m, (w.q[7] >> 4) & m);
    if (u4 == 0) {
      // 6-bit scales and mins, unpacked bytewise by the rule of
      // src/kernels/x86/kernels256.c:105-125
      const uint32_t S0 = w.hdr[1], S1 = w.hdr[2], S2 = w.hdr[3];
      const uint32_t sc_lo = S0 & 0x3F3F3F3Fu, mn_lo = S1 & 0x3F3F3F3Fu;
      const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
      const uint32_t mn_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
      sm.wsc[row][0] = sc_lo;
      sm.wsc[row][1] = sc_hi;
      uint8_t* mp = (uint8_t*)&sm.wmn[row][0];
      st16(mp, f16_pair(mn_lo & 255u), f16_pair((mn_lo >> 8) & 255u), f16_pair((mn_lo >> 16) & 255u),
           f16_pair(mn_lo >> 24));
      st16(mp + 16, f16_pair(mn_hi & 255u), f16_pair((mn_hi >> 8) & 255u), f16_pair((mn_hi >> 16) & 255u),
           f16_pair(mn_hi >> 24));
      sm.wd[row] = h2f(w.hdr[0]);
      sm.wdmin[row] = h2f(w.hdr[0] >> 16);
    }
  } else if constexpr (TT == TT_Q5_K) {
    // nibble + 16 * high bit (src/kernels/x86/kernels256.c:188-198)
    const uint32_t m = 0x0F0F0F0Fu, s0 = 2u * (uint32_t)u4;
    uint32_t lo[8], hi[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lo[i] = (w.q[i] & m) | (((w.qh[i] >> s0) & 0x01010101u) << 4);
      hi[i] = ((w.q[i] >> 4) & m) | (((w.qh[i] >> (s0 + 1)) & 0x01010101u) << 4);
    }
    st16(dst, lo[0], lo[1], lo[2], lo[3]);
    st16(dst + 16, lo[4], lo[5], lo[6], lo[7]);
    st16(dst + 32, hi[0], hi[1], hi[2], hi[3]);
    st16(dst + 48, hi[4], hi[5], hi[6], hi[7]);
    if (u4 == 0) {
      const uint32_t S0 = w.hdr[1], S1 = w.hdr[2], S2 = w.hdr[3];
      const uint32_t sc_lo = S0 & 0x3F3F3F3Fu, mn_lo = S1 & 0x3F3F3F3Fu;
      const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
      const uint32_t mn_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
      sm.wsc[row][0] = sc_lo;
      sm.wsc[row][1] = sc_hi;
      uint8_t* mp = (uint8_t*)&sm.wmn[row][0];
      st16(mp, f16_pair(mn_lo & 255u), f16_pair((mn_lo >> 8) & 255u), f16_pair((mn_lo >> 16) & 255u),
           f16_pair(mn_lo >> 24));
      st16(mp + 16, f16_pair(mn_hi & 255u), f16_pair((mn_hi >> 8) & 255u), f16_pair((mn_hi >> 16) & 255u),
           f16_pair(mn_hi >> 24));
      sm.wd[row] = h2f(w.hdr[0]);
      sm.wdmin[row] = h2f(w.hdr[0] >> 16);
    }
  } else if constexpr (TT == TT_IQ4_XS) {
    // blocks 2u4 and 2u4+1: codebook values as for IQ4_NL, scale bytes ls - 32
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const uint32_t* q = w.q + 4 * b;
      st16(dst + 32 * b, iq4_lo(q[0]), iq4_lo(q[1]), iq4_lo(q[2]), iq4_lo(q[3]));
      st16(dst + 32 * b + 16, iq4_hi(q[0]), iq4_hi(q[1]), iq4_hi(q[2]), iq4_hi(q[3]));
    }
    const uint32_t sh = w.h0 >> 16, sl = (w.sl >> (8 * u4)) & 0xFFu;
    const int ls0 = (int)((sl & 15u) | (((sh >> (4 * u4)) & 3u) << 4));
    const int ls1 = (int)((sl >> 4) | (((sh >> (4 * u4 + 2)) & 3u) << 4));
    uint8_t* sp = (uint8_t*)&sm.wsc[row][0] + 2 * u4;
    sp[0] = (uint8_t)(ls0 - 32);
    sp[1] = (uint8_t)(ls1 - 32);
    if (u4 == 0) sm.wd[row] = h2f(w.h0);
  } else if constexpr (iq3(TT)) {
    // signed grid values of sub-blocks 2u4 and 2u4+1 (Unit<>::sub's decode),
    // their scale bytes 2 ls + 1; IQ3_XXS folds its 1/4 into d (exact)
    uint32_t v[16];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        const uint32_t qq = w.q[2 * b + (l >> 1)] >> (16 * (l & 1));
        uint32_t e1, e2;
        uint2 m;
        if constexpr (TT == TT_IQ3_XXS) {
          e1 = g_iq3_grid[qq & 255u];
          e2 = g_iq3_grid[(qq >> 8) & 255u];
          m = g_iq3_sign[(w.aux[b] >> (7 * l)) & 127u];
        } else {
          const uint32_t qh = w.qh >> (8 * b);
          e1 = Unit<TT_IQ3_S>::entry(qq, qh, 2 * l);
          e2 = Unit<TT_IQ3_S>::entry(qq >> 8, qh, 2 * l + 1);
          const uint32_t s8 = w.sg[b] >> (8 * l);
          m = make_uint2(sign_bytes4(s8), sign_bytes4(s8 >> 4));
        }
        v[8 * b + 2 * l] = apply_mask4(e1, m.x);
        v[8 * b + 2 * l + 1] = apply_mask4(e2, m.y);
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) st16(dst + 16 * i, v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    uint8_t* sp = (uint8_t*)&sm.wsc[row][0] + 2 * u4;
    if constexpr (TT == TT_IQ3_XXS) {
      sp[0] = (uint8_t)(2 * (w.aux[0] >> 28) + 1);
      sp[1] = (uint8_t)(2 * (w.aux[1] >> 28) + 1);
      if (u4 == 0) sm.wd[row] = h2f(w.d) * 0.25f;
    } else {
      sp[0] = (uint8_t)(2 * (w.sc & 15u) + 1);
      sp[1] = (uint8_t)(2 * (w.sc >> 4) + 1);
      if (u4 == 0) sm.wd[row] = h2f(w.d);
    }
  } else if constexpr (TT == TT_Q3_K) {
    // unit c = values 64c..64c+63: half jj of it is shift g = 2(c&1) + jj of
    // qs[32h..] with h = c >> 1; value = q2 - 4 unless its hmask bit 4h+g is
    // set (kernels256.c:162-177): q2 | 0xFC per byte where the bit is clear
    const int h = u4 >> 1;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int g = 2 * (u4 & 1) + jj;
      uint32_t v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t q2 = (w.q[i] >> (2 * g)) & 0x03030303u;
        const uint32_t hb = (w.hm[i] >> (4 * h + g)) & 0x01010101u;
        v[i] = q2 | ((hb ^ 0x01010101u) * 0xFCu);
      }
      st16(dst + 32 * jj, v[0], v[1], v[2], v[3]);
      st16(dst + 32 * jj + 16, v[4], v[5], v[6], v[7]);
    }
    // group scales 4c..4c+3: the unpacked 6-bit values (kernels256.c:129-151) - 32
    const uint32_t base = (u4 & 1) ? w.s1 : w.s0;
    const uint32_t scw = ((u4 >= 2 ? (base >> 4) : base) & 0x0F0F0F0Fu) | (((w.s2 >> (2 * u4)) & 0x03030303u) << 4);
    sm.wsc[row][u4] = q6_minus32(scw);
    if (u4 == 0) sm.wd[row] = h2f(w.d);
  } else if constexpr (TT == TT_Q2_K) {
    // unit c = values 64c..64c+63: half jj is shift j = 2(c&1) + jj of
    // qs[32k..] with k = c >> 1 (kernels256.c:153-160)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * (u4 & 1) + jj;
      uint32_t v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = (w.q[i] >> (2 * j)) & 0x03030303u;
      st16(dst + 32 * jj, v[0], v[1], v[2], v[3]);
      st16(dst + 32 * jj + 16, v[4], v[5], v[6], v[7]);
    }
    // groups 4c..4c+3: scale = low nibble, min = high nibble
    sm.wsc[row][u4] = w.sc & 0x0F0F0F0Fu;
#pragma unroll
    for (int k = 0; k < 4; ++k) sm.wmn[row][4 * u4 + k] = (_Float16)(float)((w.sc >> (8 * k + 4)) & 15u);
    if (u4 == 0) {
      sm.wd[row] = h2f(w.dd & 0xFFFFu);
      sm.wdmin[row] = h2f(w.dd >> 16);
    }
  } else {  // Q6_K: unit (h, lh) holds values 128h + 32q + 16lh + (0..15), q = 0..3
    const int h = (u4 >> 1) & 1, lh = u4 & 1;
    uint32_t v[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t la = w.la[i], lb = w.lb[i], qh = w.qh[i];
      v[0][i] = q6_minus32((la & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4));
      v[1][i] = q6_minus32((lb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u));
      v[2][i] = q6_minus32(((la >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u));
      v[3][i] = q6_minus32(((lb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u));
    }
    uint8_t* rowp = sm.bq + row * kQS;
#pragma unroll
    for (int q = 0; q < 4; ++q) st16(rowp + 128 * h + 32 * q + 16 * lh, v[q][0], v[q][1], v[q][2], v[q][3]);
    // scales sc[8h + lh + 2q]: bytes 0 and 2 of sc01 and sc23
    uint8_t* sp = (uint8_t*)&sm.wsc[row][0] + 8 * h + lh;
    sp[0] = (uint8_t)w.sc01;
    sp[2] = (uint8_t)(w.sc01 >> 16);
    sp[4] = (uint8_t)w.sc23;
    sp[6] = (uint8_t)(w.sc23 >> 16);
    if (u4 == 0) sm.wd[row] = h2f(w.d);
  }
}

// ---- staging: activations --------------------------------------------------------------
// The 32-value formats take Q8_0 activations (two blocks per unit); the
// K-quants take a Q8_K quarter in plain value order: values 64*u4 .. 64*u4+63.
template <int TT>
using MmqAct = typename std::conditional<act32(TT), ActPair, ActQ8K>::type;

template <int TT>
__device__ __forceinline__ MmqAct<TT> load_act(const uint8_t* arow, int u) {
  if constexpr (act32(TT)) return act_pair_ref(arow, u);
  else return Unit<TT_Q4_K>::load_a(arow, u);
}

template <int TT, class SM>
__device__ __forceinline__ void emit_a(SM& sm, const MmqAct<TT>& a, int tok, int u4) {
  uint8_t* dst = sm.aq + tok * kQS + 64 * u4;
  if constexpr (act32(TT)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) st16(dst + 16 * i, a.q[4 * i], a.q[4 * i + 1], a.q[4 * i + 2], a.q[4 * i + 3]);
    sm.ad[2 * u4][tok] = a.d0;
    sm.ad[2 * u4 + 1][tok] = a.d1;
    if constexpr (TT == TT_Q4_1) {
      int y0 = 0, y1 = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y0 = dot4(0x01010101u, a.q[i], y0);
        y1 = dot4(0x01010101u, a.q[8 + i], y1);
      }
      sm.ay[2 * u4][tok] = a.d0 * (float)y0;
      sm.ay[2 * u4 + 1][tok] = a.d1 * (float)y1;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) st16(dst + 16 * i, a.y[4 * i], a.y[4 * i + 1], a.y[4 * i + 2], a.y[4 * i + 3]);
    if constexpr (TT == TT_Q4_K || TT == TT_Q5_K || TT == TT_Q2_K) {
      _Float16* bp = &sm.abs[tok][4 * u4];
#pragma unroll
      for (int i = 0; i < 4; ++i) bp[i] = (_Float16)(float)a.bs[i];
    }
    if (u4 == 0) sm.ady[tok] = a.d;
  }
}

// ---- tile output -----------------------------------------------------------------------
// Lanes 0..31 of a wave write 32 consecutive rows of one token per element.
// Split over K (ksplit > 1): each slice's workgroup stores its partial tile in
// part[(tile * ksplit + slice) * tile_elems + i] (i: the thread's element in
// accumulator order, so the stores are coalesced) and the last workgroup of
// the tile adds the slices in slice order (sk_* hand-off, qhip_device.hpp):
// the output does not depend on which slice finished last.  The last
// workgroup's loads of several slices go out together (up to 64 values per
// lane in flight): each batch costs one memory latency, and a grid cut into
// 20-30 slices would otherwise wait one latency per slice.  NEL < 16: only the
// first NEL accumulator elements hold real tokens (the few-token kernels);
// the rest are neither handed off nor written.
template <int NA, int NB, int NW, int NEL = 16>
__device__ __forceinline__ void mmq_write_tile(f32x16 (&acc)[NA][NB], float* __restrict__ Y, int rows, int tokens,
                                               int r0, int t0, int rb0, int tb0, int tile, int ksplit, int ks,
                                               float* __restrict__ part, unsigned* __restrict__ cnt) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 31, lh = lane >> 5;
  if (ksplit > 1) {
    constexpr long TS = (long)NW * NA * NB * 1024;  // elements per tile
    const long mine = (long)wv * NA * NB * 1024 + lane;
    float* pp = part + ((long)tile * ksplit + ks) * TS + mine;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int e = 0; e < NEL; ++e) sk_store(pp + ((a * NB + b) * 16 + e) * 64, acc[a][b][e]);
    if (!sk_arrive(cnt + tile, (unsigned)ksplit)) return;
    const float* base = part + (long)tile * ksplit * TS + mine;
    // in slice order, U slices' loads at a time (a batch past the last slice
    // re-reads the last one and drops it)
    constexpr int PER = NA * NB * NEL, U = PER >= 64 ? 1 : 64 / PER;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;
    for (int q0 = 0; q0 < ksplit; q0 += U) {
      float t[U][NA][NB][NEL];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float* pq = base + (q0 + u < ksplit ? q0 + u : ksplit - 1) * TS;
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int e = 0; e < NEL; ++e) t[u][a][b][e] = sk_load(pq + ((a * NB + b) * 16 + e) * 64);
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (q0 + u < ksplit)
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
              for (int e = 0; e < NEL; ++e) acc[a][b][e] += t[u][a][b][e];
    }
    sk_reset(cnt + tile);
  }
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      const int row = r0 + rb0 + 32 * b + li;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int tok = t0 + tb0 + 32 * a + 8 * (e >> 2) + 4 * lh + (e & 3);
        if (row < rows && tok < tokens) Y[(long)tok * rows + row] = acc[a][b][e];
      }
    }
}

// ---- the kernel -------------------------------------------------------------------------
// SPLIT = false: the launch is not cut over K (ksplit == 1); without the
// hand-off's code the kernel needs fewer registers (Q8_0 64 x 64: 156 VGPRs
// against 171, three waves per SIMD instead of two).
template <int TT, int BT, int BR, int NT = 256, bool SPLIT = true>
__global__ __launch_bounds__(NT) void k_mmq(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ,
                                              float* __restrict__ Y, int rows, int tokens, long row_bytes,
                                              long act_bytes, int upr, int ntile_t, int ksplit, int cps,
                                              float* __restrict__ part, unsigned* __restrict__ cnt) {
  if constexpr (!SPLIT) ksplit = 1;
  grid_prologue<TT>();
  constexpr bool K32 = act32(TT);
  // waves: 2 x 2 over (tokens, rows), or stacked along rows for a 32-token
  // tile (four waves for 128 rows, two for 64)
  constexpr int NW = NT / 64;
  constexpr int WT = BT >= 64 ? 2 : 1, WR = NW / WT;
  constexpr int NA = BT / (32 * WT), NB = BR / (32 * WR);
  static_assert(NA >= 1 && NB >= 1, "tile too small for the wave layout");
  __shared__ MmqSmem<TT, BT, BR> sm;

  // Tile order: the hardware deals workgroups round-robin to the 8 XCDs;
  // give each XCD a contiguous run of row tiles (all their token tiles), so
  // a weight chunk is fetched into one XCD's L2 and reused there.  With
  // ksplit > 1 the K range is cut into ksplit slices of cps chunks; each
  // workgroup adds its slice's partial tile into the zero-filled output.
  const int G = gridDim.x;
  int g = blockIdx.x;
  if ((G & 7) == 0) g = (g & 7) * (G >> 3) + (g >> 3);
  const int ks = g % ksplit;
  g /= ksplit;
  const int r0 = (g / ntile_t) * BR, t0 = (g % ntile_t) * BT;

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 31, lh = lane >> 5;
  const int tb0 = (wv % WT) * (BT / WT), rb0 = (wv / WT) * (BR / WR);

  f32x16 acc[NA][NB];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;

  // Thread tid stages weight units tid + NT*i (row q>>2, unit q&3) and the
  // activation units likewise (threads 0..4*BT-1 only when the tile has
  // fewer tokens than NT/4); rows / tokens past the end re-read the last one.
  constexpr int UW = 4 * BR / NT, UA = 4 * BT >= NT ? 4 * BT / NT : 1;
  static_assert(UW >= 1, "too few rows for the workgroup");
  const bool a_on = 4 * BT >= NT || tid < 4 * BT;
  typename Unit<TT>::W wreg[UW];
  MmqAct<TT> areg[UA];
  const uint8_t* wrow[UW];
  const uint8_t* arow[UA];
#pragma unroll
  for (int i = 0; i < UW; ++i) {
    const int row = (tid + NT * i) >> 2;
    wrow[i] = W + (long)(r0 + row < rows ? r0 + row : rows - 1) * row_bytes;
  }
#pragma unroll
  for (int i = 0; i < UA; ++i) {
    const int tok = (tid + NT * i) >> 2;
    arow[i] = XQ + (long)(t0 + tok < tokens ? t0 + tok : tokens - 1) * act_bytes;
  }
  const int u4 = tid & 3;
  const int nchunks_all = (upr + 3) >> 2;
  const int ch_begin = ks * cps;
  const int nchunks = ch_begin + cps < nchunks_all ? ch_begin + cps : nchunks_all;
  auto load_chunk = [&](int ch) {
    if (4 * ch + u4 < upr) {
#pragma unroll
      for (int i = 0; i < UW; ++i) wreg[i] = Unit<TT>::load_w(wrow[i], 4 * ch + u4);
      if (a_on) {
#pragma unroll
        for (int i = 0; i < UA; ++i) areg[i] = load_act<TT>(arow[i], 4 * ch + u4);
      }
    }
  };
  if (ch_begin < nchunks) load_chunk(ch_begin);
  for (int ch = ch_begin; ch < nchunks; ++ch) {
    const int nu = upr - 4 * ch < 4 ? upr - 4 * ch : 4;  // units in this chunk
    __syncthreads();  // the previous chunk's fragments have been read
    if (u4 < nu) {
#pragma unroll
      for (int i = 0; i < UW; ++i) emit_w<TT, BT, BR>(sm, wreg[i], (tid + NT * i) >> 2, u4);
      if (a_on) {
#pragma unroll
        for (int i = 0; i < UA; ++i) emit_a<TT>(sm, areg[i], (tid + NT * i) >> 2, u4);
      }
    }
    __syncthreads();
    if (ch + 1 < nchunks) load_chunk(ch + 1);  // in flight during this chunk's MFMAs

    if constexpr (K32) {
      i32x16 bias;
#pragma unroll
      for (int e = 0; e < 16; ++e) bias[e] = kBiasBits;
      // opaque to the optimizer: the bias stays in 16 registers as every
      // MFMA's accumulator input (instead of being re-created per MFMA)
      asm volatile("" : "+v"(bias));
      // issue: fragments of block s and its MFMAs; finish: scale and
      // accumulate block s.  Software-pipelined: block s+1's MFMAs are issued
      // before block s is scaled, so the matrix core and the VALU overlap.
      auto issue = [&](int s, i32x16 (&c)[NA][NB], float (&dw)[NB]) {
        i32x4 af[NA], bf[NB];
#pragma unroll
        for (int a = 0; a < NA; ++a)
          af[a] = *(const i32x4*)(sm.aq + (tb0 + 32 * a + li) * kQS + 32 * s + 16 * lh);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          bf[b] = *(const i32x4*)(sm.bq + (rb0 + 32 * b + li) * kQS + 32 * s + 16 * lh);
          dw[b] = sm.wd[s][rb0 + 32 * b + li];
        }
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b) c[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bf[b], bias, 0, 0, 0);
      };
      auto finish = [&](int s, const i32x16 (&c)[NA][NB], const float (&dw)[NB]) {
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          f32x4 da[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) da[q] = *(const f32x4*)&sm.ad[s][tb0 + 32 * a + 8 * q + 4 * lh];
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const float cw = -kBias * dw[b];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              // (a scalar copy first: bit-casting the vector element
              // expression c[e] directly reads element 0 for every e)
              const int ce = c[a][b][e];
              const float t = __builtin_fmaf(__int_as_float(ce), dw[b], cw);
              acc[a][b][e] = __builtin_fmaf(t, da[e >> 2][e & 3], acc[a][b][e]);
            }
          }
        }
        if constexpr (TT == TT_Q4_1) {
          // the mins: acc += m[r] * (dy * sumy)[t]
          float wm[NB];
#pragma unroll
          for (int b = 0; b < NB; ++b) wm[b] = sm.wm[s][rb0 + 32 * b + li];
#pragma unroll
          for (int a = 0; a < NA; ++a) {
            f32x4 ay[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) ay[q] = *(const f32x4*)&sm.ay[s][tb0 + 32 * a + 8 * q + 4 * lh];
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[a][b][e] = __builtin_fmaf(wm[b], ay[e >> 2][e & 3], acc[a][b][e]);
          }
        }
      };
      i32x16 c0[NA][NB], c1[NA][NB];
      float dw0[NB], dw1[NB];
      if (nu == 4) {
        issue(0, c0, dw0);
#pragma unroll
        for (int s2 = 0; s2 < 8; s2 += 2) {
          issue(s2 + 1, c1, dw1);
          finish(s2, c0, dw0);
          if (s2 + 2 < 8) issue(s2 + 2, c0, dw0);
          finish(s2 + 1, c1, dw1);
        }
      } else {
        for (int s2 = 0; s2 < 2 * nu; ++s2) {
          issue(s2, c0, dw0);
          finish(s2, c0, dw0);
        }
      }
    } else if constexpr (TT == TT_Q4_K || TT == TT_Q5_K || TT == TT_IQ4_XS || iq3(TT)) {
      i32x16 isum[NA][NB];
      const i32x16 zero = {};
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) isum[a][b] = zero;
      uint32_t scw[NB][2];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        scw[b][0] = sm.wsc[rb0 + 32 * b + li][0];
        scw[b][1] = sm.wsc[rb0 + 32 * b + li][1];
      }
      if constexpr (TT == TT_Q4_K) {
        // Split scales: the 6-bit sub-block scale sc = 8 sh + sl (sh, sl <= 7),
        // so sh*q and sl*q (q <= 15) fit int8.  Both products are formed on the
        // weight fragment (bytewise: a 16-bit lane multiply of two packed
        // bytes carries nothing across them, each product being < 256), and
        // two MFMA chains accumulate the whole super-block with the scales
        // already applied: isum = 8 C_hi + C_lo, the same exact integer as
        // sum_s sc_s * sumi_s, with no per-sub-block integer scaling.
        i32x16 chi[NA][NB], clo[NA][NB];
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            chi[a][b] = zero;
            clo[a][b] = zero;
          }
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          i32x4 af[NA], bh[NB], bl[NB];
#pragma unroll
          for (int a = 0; a < NA; ++a) af[a] = *(const i32x4*)(sm.aq + (tb0 + 32 * a + li) * kQS + 32 * s + 16 * lh);
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const i32x4 q = *(const i32x4*)(sm.bq + (rb0 + 32 * b + li) * kQS + 32 * s + 16 * lh);
            const uint32_t sc = (scw[b][s >> 2] >> (8 * (s & 3))) & 63u;
            const u16x2 mh = {(uint16_t)(sc >> 3), (uint16_t)(sc >> 3)};
            const u16x2 ml = {(uint16_t)(sc & 7u), (uint16_t)(sc & 7u)};
            // (scalar copies first: bit-casting a vector element expression
            // reads element 0 for every index)
            const uint32_t q0 = q.x, q1 = q.y, q2 = q.z, q3 = q.w;
            const uint32_t h0 = __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, q0) * mh));
            const uint32_t h1 = __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, q1) * mh));
            const uint32_t h2 = __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, q2) * mh));
            const uint32_t h3 = __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, q3) * mh));
            const uint32_t l0 = __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, q0) * ml));
            const uint32_t l1 = __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, q1) * ml));
            const uint32_t l2 = __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, q2) * ml));
            const uint32_t l3 = __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, q3) * ml));
            bh[b] = i32x4{(int)h0, (int)h1, (int)h2, (int)h3};
            bl[b] = i32x4{(int)l0, (int)l1, (int)l2, (int)l3};
          }
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
              chi[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bh[b], chi[a][b], 0, 0, 0);
              clo[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bl[b], clo[a][b], 0, 0, 0);
            }
        }
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e) isum[a][b][e] = 8 * chi[a][b][e] + clo[a][b][e];
      } else {
      // pipelined as in the 32-value path: sub-block s+1's MFMAs are issued
      // before sub-block s's integer scaling
      auto issue = [&](int s, i32x16 (&c)[NA][NB]) {
        i32x4 af[NA], bf[NB];
#pragma unroll
        for (int a = 0; a < NA; ++a) af[a] = *(const i32x4*)(sm.aq + (tb0 + 32 * a + li) * kQS + 32 * s + 16 * lh);
#pragma unroll
        for (int b = 0; b < NB; ++b) bf[b] = *(const i32x4*)(sm.bq + (rb0 + 32 * b + li) * kQS + 32 * s + 16 * lh);
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b) c[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bf[b], zero, 0, 0, 0);
      };
      auto finish = [&](int s, const i32x16 (&c)[NA][NB]) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const uint32_t sb = scw[b][s >> 2] >> (8 * (s & 3));
          const int sc = TT == TT_IQ4_XS ? sext8(sb) : (int)(sb & 0xFFu);
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int e = 0; e < 16; ++e) isum[a][b][e] += sc * sext24(c[a][b][e]);
        }
      };
      i32x16 c0[NA][NB], c1[NA][NB];
      issue(0, c0);
#pragma unroll
      for (int s = 0; s < 8; s += 2) {
        issue(s + 1, c1);
        finish(s, c0);
        if (s + 2 < 8) issue(s + 2, c0);
        finish(s + 1, c1);
      }
      }
      if constexpr (TT == TT_IQ4_XS || iq3(TT)) {
        // no mins: acc += (d * dy) * isum  (iq_kernels.c:967-1001, one
        // rounding of the exact super-block integer instead of one per block)
        f32x4 dy[NA][4];
        float d[NB];
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int q = 0; q < 4; ++q) dy[a][q] = *(const f32x4*)&sm.ady[tb0 + 32 * a + 8 * q + 4 * lh];
#pragma unroll
        for (int b = 0; b < NB; ++b) d[b] = sm.wd[rb0 + 32 * b + li];
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e)
              acc[a][b][e] = __builtin_fmaf(d[b] * dy[a][e >> 2][e & 3], (float)isum[a][b][e], acc[a][b][e]);
      } else {
      // mins: summs[t][r] = sum_j bsum[t][j] * min[r][j/2], exact in the f16 MFMA
      f16x8 am[NA], bm[NB];
      f32x4 dy[NA][4];
      float d[NB], ndm[NB];
#pragma unroll
      for (int a = 0; a < NA; ++a) {
        am[a] = *(const f16x8*)&sm.abs[tb0 + 32 * a + li][8 * lh];
#pragma unroll
        for (int q = 0; q < 4; ++q) dy[a][q] = *(const f32x4*)&sm.ady[tb0 + 32 * a + 8 * q + 4 * lh];
      }
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        bm[b] = *(const f16x8*)&sm.wmn[rb0 + 32 * b + li][8 * lh];
        d[b] = sm.wd[rb0 + 32 * b + li];
        ndm[b] = -sm.wdmin[rb0 + 32 * b + li];
      }
      const f32x16 fz = {};
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const f32x16 cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[a], bm[b], fz, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const float inner = __builtin_fmaf(d[b], (float)isum[a][b][e], ndm[b] * cm[e]);
            acc[a][b][e] = __builtin_fmaf(dy[a][e >> 2][e & 3], inner, acc[a][b][e]);
          }
        }
      }
    } else {  // Q6_K
      i32x16 isum[NA][NB];
      const i32x16 zero = {};
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) isum[a][b] = zero;
      uint32_t scw[NB][4];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const uint4 v = *(const uint4*)&sm.wsc[rb0 + 32 * b + li][0];
        scw[b][0] = v.x; scw[b][1] = v.y; scw[b][2] = v.z; scw[b][3] = v.w;
      }
      // pipelined: group g+1's MFMAs are issued before group g is scaled
      auto issue = [&](int gq, i32x16 (&c)[NA][NB]) {
        long af[NA], bf[NB];
#pragma unroll
        for (int a = 0; a < NA; ++a) af[a] = *(const i64x1_a8*)(sm.aq + (tb0 + 32 * a + li) * kQS + 16 * gq + 8 * lh);
#pragma unroll
        for (int b = 0; b < NB; ++b) bf[b] = *(const i64x1_a8*)(sm.bq + (rb0 + 32 * b + li) * kQS + 16 * gq + 8 * lh);
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b) c[a][b] = __builtin_amdgcn_mfma_i32_32x32x16_i8(af[a], bf[b], zero, 0, 0, 0);
      };
      auto finish = [&](int gq, const i32x16 (&c)[NA][NB]) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const int sc = sext8(scw[b][gq >> 2] >> (8 * (gq & 3)));
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int e = 0; e < 16; ++e) isum[a][b][e] += sc * sext24(c[a][b][e]);
        }
      };
      i32x16 c0[NA][NB], c1[NA][NB];
      issue(0, c0);
#pragma unroll
      for (int gq = 0; gq < 16; gq += 2) {
        issue(gq + 1, c1);
        finish(gq, c0);
        if (gq + 2 < 16) issue(gq + 2, c0);
        finish(gq + 1, c1);
      }
      f32x4 dy[NA][4];
      float d[NB];
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int q = 0; q < 4; ++q) dy[a][q] = *(const f32x4*)&sm.ady[tb0 + 32 * a + 8 * q + 4 * lh];
#pragma unroll
      for (int b = 0; b < NB; ++b) d[b] = sm.wd[rb0 + 32 * b + li];
      if constexpr (TT == TT_Q2_K) {
        // mins: summs[t][r] = sum_g bsum[t][g] * min[r][g], exact in the f16
        // MFMA (|bsum| <= 2032, min <= 15, 16 groups: < 2^24)
        // (kernels256.c:232-257: dall * isum - dmin * summs)
        f16x8 am[NA], bm[NB];
        float ndm[NB];
#pragma unroll
        for (int a = 0; a < NA; ++a) am[a] = *(const f16x8*)&sm.abs[tb0 + 32 * a + li][8 * lh];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          bm[b] = *(const f16x8*)&sm.wmn[rb0 + 32 * b + li][8 * lh];
          ndm[b] = -sm.wdmin[rb0 + 32 * b + li];
        }
        const f32x16 fz = {};
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            const f32x16 cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[a], bm[b], fz, 0, 0, 0);
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const float inner = __builtin_fmaf(d[b], (float)isum[a][b][e], ndm[b] * cm[e]);
              acc[a][b][e] = __builtin_fmaf(dy[a][e >> 2][e & 3], inner, acc[a][b][e]);
            }
          }
      } else {
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int e = 0; e < 16; ++e)
              acc[a][b][e] = __builtin_fmaf(d[b] * dy[a][e >> 2][e & 3], (float)isum[a][b][e], acc[a][b][e]);
      }
    }
  }

  mmq_write_tile<NA, NB, NW>(acc, Y, rows, tokens, r0, t0, rb0, tb0, g, ksplit, ks, part, cnt);
}

// ---- split-K for small grids ----------------------------------------------------------
// With fewer than two tile workgroups per CU the K loop of each tile is one
// long dependent chain and the GPU idles.  For at most two token tiles (where
// the output is small) K is cut into slices of at least `min_chunks` chunks,
// aiming at about four workgroups per CU.  The slices' partial tiles go to a
// caller workspace and the last workgroup of each tile adds them in slice
// order (mmq_write_tile), so the output is the same on every run.  Without a
// workspace large enough for the partials, K is not split.
static int mmq_ksplit_for(const GemvArgs& g, int bt, int br, int nchunks, int min_chunks) {
  const long ntt = (g.tokens + bt - 1) / bt;
  const long tiles = (long)((g.rows + br - 1) / br) * ntt;
  if (tiles >= 512 || ntt > 2 || nchunks < 2 * min_chunks) return 1;
  const long want = (1024 + tiles - 1) / tiles;
  const int cap = nchunks / min_chunks;
  return (int)(want < cap ? want : cap);
}

// Slices for a launch of `tiles` tiles of a kernel that holds two workgroups
// per CU (the weights-direct and image MMQs: their registers allow two waves
// per SIMD).  A grid of 1.25 rounds of resident workgroups spends a whole
// round at a quarter of the GPU; cutting K evens the rounds at the price of
// the partial tiles' traffic.  Below one round: the smallest count of 1..4
// whose grid fills its rounds at least 80%, else the fullest.  From one to
// two rounds: the count with the best fill less 0.06 per extra slice.  Two
// rounds or more: unsplit.  Measured on MI355X (config 5 Q4_K
// weights-direct, us at 1 / 2 / 3 / 4 slices): T = 128 57 / 54 / 46 / 50;
// T = 256 92 / 84 / 78 / 84; T = 384 110 / 114 / 113 / 120; T = 512 144 /
// 147 / 152 / 162 (two slices also tripled the launch's HBM writes); T =
// 1024 256 / 294 / 310 / 346 -- the rule picks the fastest count at each
// (3, 3, 1, 1, 1).
extern "C" int qhip_gpu_cu_count(void);
static int mmq_round_slices(long tiles, int nchunks, int min_chunks) {
  if (tiles > kSkMaxTiles) return 1;
  const int cus = qhip_gpu_cu_count();
  const long cap = 2L * (cus > 0 ? cus : 256);
  if (tiles >= 2 * cap) return 1;
  const double penalty = tiles >= cap ? 0.06 : 0.0;
  int best = 1;
  double best_s = -1.0;
  for (int ks = 1; ks <= 4; ++ks) {
    if (ks > 1 && nchunks / ks < min_chunks) break;
    const long w = tiles * ks, rounds = (w + cap - 1) / cap;
    const double fill = (double)w / (double)(rounds * cap);
    if (penalty == 0.0 && fill >= 0.8) return ks;
    const double score = fill - penalty * (ks - 1);
    if (score > best_s) {
      best_s = score;
      best = ks;
    }
  }
  return best;
}

// Slices actually launched for a requested ksplit (no empty slice).
static int mmq_slices(int nchunks, int ksplit) {
  if (ksplit < 1) ksplit = 1;
  if (ksplit > nchunks) ksplit = nchunks;
  const int cps = (nchunks + ksplit - 1) / ksplit;
  return (nchunks + cps - 1) / cps;
}

// Workspace of a split launch: the tile counters, then the partial tiles.
static long mmq_split_bytes(const GemvArgs& g, int bt, int br, int slices) {
  if (slices <= 1) return 0;
  const long tiles = (long)((g.rows + br - 1) / br) * ((g.tokens + bt - 1) / bt);
  return kSkCountBytes + 4L * slices * tiles * bt * br;
}

// ---- MMQ on a prepared weight image (Q4_K; Q6_K's image is the plane image below) -----
// The Q4_K integer sub-scales are folded into the quantized values once, at
// weight-load time: p = sc * q (0..945), split exactly into two int8 planes
// p = 2^7 hi + lo (hi 0..7, lo 0..127).  A super-block then needs no
// per-group scaling: the 32x32x32 int8 MFMAs of both planes accumulate the
// whole super-block, and isum = (hi_sum << 7) + lo_sum is the reference's
// integer (kernels256.c:474-498) exactly.  Twice the MFMAs, a sixth of the
// VALU work per output.  The image costs 560 bytes per 256 values (3.9x the
// GGUF bytes).
//
// Image layout (two regions, both 16-byte aligned):
//   planes  [row][super-block] 512 bytes: hi plane [0, 256), lo plane [256, 512),
//           values in order
//   headers [row][super-block] 48 bytes: min of each 16-value group as f16
//           (min[j/2]) [0, 32), d f32 [32, 36), dmin f32 [36, 40)
template <int TT>
__host__ __device__ constexpr int img_hdr_bytes() { return 48; }
__host__ __device__ constexpr int img_shift(int) { return 7; }
// one thread per (row, super-block, 16-value group)
template <int TT>
__global__ __launch_bounds__(256) void k_mmq_prepare(const uint8_t* __restrict__ W, uint8_t* __restrict__ IMG,
                                                      long nsb_total, long row_bytes, int nsb) {
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= nsb_total * 16) return;
  const int g = (int)(gid & 15);
  const long sbi = gid >> 4;  // row * nsb + sb
  const long row = sbi / nsb, sb = sbi % nsb;
  const uint8_t* blk = W + row * row_bytes + sb * 144;
  uint8_t* ib = IMG + sbi * 512;
  uint8_t* hb = IMG + nsb_total * 512 + sbi * img_hdr_bytes<TT>();
  uint32_t hi[4] = {0, 0, 0, 0}, lo[4] = {0, 0, 0, 0};
  static_assert(TT == TT_Q4_K, "the Q6_K image is the plane image");
  {
    const int sub = g >> 1;  // 32-value sub-block, src/kernels/x86/kernels256.c:105-125
    const uint8_t* s12 = blk + 4;
    int sc, m;
    if (sub < 4) {
      sc = s12[sub] & 63;
      m = s12[sub + 4] & 63;
    } else {
      sc = (s12[sub + 4] & 15) | ((s12[sub - 4] >> 6) << 4);
      m = (s12[sub + 4] >> 4) | ((s12[sub] >> 6) << 4);
    }
    (void)m;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int l = 16 * (g & 1) + i;
      const uint32_t qb = blk[16 + 32 * (sub >> 1) + l];
      const int q = (int)((sub & 1) ? (qb >> 4) : (qb & 15u));
      const int pv = sc * q;
      hi[i >> 2] |= (uint32_t)(pv >> 7) << (8 * (i & 3));
      lo[i >> 2] |= (uint32_t)(pv & 127) << (8 * (i & 3));
    }
    if (g == 0) {
      // min of every 16-value group j: min[j/2], as f16 for the mins MFMA
      uint32_t mw[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int mk = k < 4 ? (s12[k + 4] & 63) : ((s12[k + 4] >> 4) | ((s12[k] >> 6) << 4));
        mw[k] = f16_pair((uint32_t)mk);
      }
      *(uint4*)(hb) = make_uint4(mw[0], mw[1], mw[2], mw[3]);
      *(uint4*)(hb + 16) = make_uint4(mw[4], mw[5], mw[6], mw[7]);
      const float d = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
      const float dmin = h2f((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
      *(uint4*)(hb + 32) = make_uint4(__float_as_uint(d), __float_as_uint(dmin), 0u, 0u);
    }
  }
  *(uint4*)(ib + 16 * g) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  *(uint4*)(ib + 256 + 16 * g) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
}

template <int TT, int BT, int BR>
struct alignas(16) ImgSmem {
  uint8_t aq[BT * kQS];
  uint8_t bqh[BR * kQS];
  uint8_t bql[BR * kQS];
  _Float16 abs[BT][16];
  _Float16 wmn[BR][16];
  float ady[BT];
  float wd[BR], wdmin[BR];
};

template <int TT, int BT, int BR>
__global__ __launch_bounds__(256) void k_mmq_img(const uint8_t* __restrict__ IMG, const uint8_t* __restrict__ XQ,
                                                  float* __restrict__ Y, int rows, int tokens, int nsb,
                                                  long act_bytes, int ntile_t, int ksplit, int cps,
                                                  float* __restrict__ part, unsigned* __restrict__ cnt) {
  constexpr int HB = img_hdr_bytes<TT>(), NH = HB / 16;
  constexpr int S = img_shift(TT);
  constexpr int NA = BT / 64, NB = BR / 64;
  constexpr int PW = BR * 32 / 256;            // 16-byte plane pieces per thread per chunk
  constexpr int PH = (BR * NH + 255) / 256;    // header pieces per thread per chunk
  constexpr int UA = BT / 64;
  __shared__ ImgSmem<TT, BT, BR> sm;

  const int G = gridDim.x;
  int g = blockIdx.x;
  if ((G & 7) == 0) g = (g & 7) * (G >> 3) + (g >> 3);  // XCD-contiguous row tiles, as k_mmq
  // K slice ks: super-blocks [ks*cps, ks*cps + cps); tiles ordered (row tile,
  // K slice, token tile), as k_mmq_wd_q4k
  const int per = ksplit * ntile_t, rt = g / per, ks = (g - rt * per) / ntile_t;
  const int tt = g - rt * per - ks * ntile_t;
  g = rt * ntile_t + tt;
  const int r0 = rt * BR, t0 = tt * BT;
  const int sb_begin = ks * cps, sb_end = sb_begin + cps < nsb ? sb_begin + cps : nsb;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int li = lane & 31, lh = lane >> 5;
  const int tb0 = (wv & 1) * (BT / 2), rb0 = (wv >> 1) * (BR / 2);

  f32x16 acc[NA][NB];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[a][b][e] = 0.0f;

  // plane piece p = tid + 256*i: row p >> 5, piece p & 31 of its 512 bytes;
  // header piece q = tid + 256*i: row q / NH, piece q % NH
  const long nsb_total = (long)rows * nsb;
  const uint8_t* hdr = IMG + nsb_total * 512;
  i32x4 wreg[PW], hreg[PH];
  const uint8_t* wsrc[PW];
  const uint8_t* hsrc[PH];
#pragma unroll
  for (int i = 0; i < PW; ++i) {
    const int p = tid + 256 * i, row = p >> 5;
    const int rg = r0 + row < rows ? r0 + row : rows - 1;
    wsrc[i] = IMG + (long)rg * nsb * 512 + 16 * (p & 31);
  }
#pragma unroll
  for (int i = 0; i < PH; ++i) {
    const int q = tid + 256 * i, row = q / NH < BR ? q / NH : BR - 1;
    const int rg = r0 + row < rows ? r0 + row : rows - 1;
    hsrc[i] = hdr + (long)rg * nsb * HB + 16 * (q % NH);
  }
  MmqAct<TT> areg[UA];
  const uint8_t* arow[UA];
#pragma unroll
  for (int i = 0; i < UA; ++i) {
    const int tok = (tid + 256 * i) >> 2;
    arow[i] = XQ + (long)(t0 + tok < tokens ? t0 + tok : tokens - 1) * act_bytes;
  }
  const int u4 = tid & 3;
  auto load_chunk = [&](int sb) {
#pragma unroll
    for (int i = 0; i < PW; ++i) wreg[i] = *(const i32x4*)(wsrc[i] + (long)sb * 512);
#pragma unroll
    for (int i = 0; i < PH; ++i)
      if (tid + 256 * i < BR * NH) hreg[i] = *(const i32x4*)(hsrc[i] + (long)sb * HB);
#pragma unroll
    for (int i = 0; i < UA; ++i) areg[i] = load_act<TT>(arow[i], 4 * sb + u4);
  };
  if (sb_begin < sb_end) load_chunk(sb_begin);
  for (int sb = sb_begin; sb < sb_end; ++sb) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < PW; ++i) {
      const int p = tid + 256 * i, row = p >> 5, k = p & 31;
      uint8_t* dst = (k < 16 ? sm.bqh + 16 * k : sm.bql + 16 * (k - 16)) + row * kQS;
      *(i32x4*)dst = wreg[i];
    }
#pragma unroll
    for (int i = 0; i < PH; ++i) {
      const int q = tid + 256 * i;
      if (q < BR * NH) {
        const int row = q / NH, k = q % NH;
        if (k < 2) {
          *(i32x4*)((uint8_t*)&sm.wmn[row][0] + 16 * k) = hreg[i];
        } else {
          sm.wd[row] = __int_as_float(hreg[i].x);
          sm.wdmin[row] = __int_as_float(hreg[i].y);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < UA; ++i) emit_a<TT>(sm, areg[i], (tid + 256 * i) >> 2, u4);
    __syncthreads();
    if (sb + 1 < sb_end) load_chunk(sb + 1);  // in flight during this chunk's MFMAs

    i32x16 chi[NA][NB], clo[NA][NB];
    const i32x16 zero = {};
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        chi[a][b] = zero;
        clo[a][b] = zero;
      }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      i32x4 af[NA], bh[NB], bl[NB];
#pragma unroll
      for (int a = 0; a < NA; ++a) af[a] = *(const i32x4*)(sm.aq + (tb0 + 32 * a + li) * kQS + 32 * s + 16 * lh);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        bh[b] = *(const i32x4*)(sm.bqh + (rb0 + 32 * b + li) * kQS + 32 * s + 16 * lh);
        bl[b] = *(const i32x4*)(sm.bql + (rb0 + 32 * b + li) * kQS + 32 * s + 16 * lh);
      }
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          chi[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bh[b], chi[a][b], 0, 0, 0);
          clo[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[a], bl[b], clo[a][b], 0, 0, 0);
        }
    }
    f32x4 dy[NA][4];
    float d[NB];
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int q = 0; q < 4; ++q) dy[a][q] = *(const f32x4*)&sm.ady[tb0 + 32 * a + 8 * q + 4 * lh];
#pragma unroll
    for (int b = 0; b < NB; ++b) d[b] = sm.wd[rb0 + 32 * b + li];
    {
      f16x8 am[NA], bm[NB];
      float ndm[NB];
#pragma unroll
      for (int a = 0; a < NA; ++a) am[a] = *(const f16x8*)&sm.abs[tb0 + 32 * a + li][8 * lh];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        bm[b] = *(const f16x8*)&sm.wmn[rb0 + 32 * b + li][8 * lh];
        ndm[b] = -sm.wdmin[rb0 + 32 * b + li];
      }
      const f32x16 fz = {};
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          const f32x16 cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am[a], bm[b], fz, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int isum = (chi[a][b][e] << S) + clo[a][b][e];
            const float inner = __builtin_fmaf(d[b], (float)isum, ndm[b] * cm[e]);
            acc[a][b][e] = __builtin_fmaf(dy[a][e >> 2][e & 3], inner, acc[a][b][e]);
          }
        }
    }
  }

  mmq_write_tile<NA, NB, 4>(acc, Y, rows, tokens, r0, t0, rb0, tb0, g, ksplit, ks, part, cnt);
}

long mmq_image_bytes(int ttype, int rows, int cols) {
  if (ttype == TT_Q6_K) return bg_image_bytes_q6k(rows, cols);
  if (ttype != TT_Q4_K || rows < 0 || cols <= 0 || cols % 256) return -1;
  return (long)rows * (cols / 256) * (512 + img_hdr_bytes<TT_Q4_K>());
}

hipError_t launch_mmq_prepare(int ttype, const void* w, long row_bytes, int rows, int cols, void* img,
                              hipStream_t s) {
  if (ttype == TT_Q6_K) return launch_bg_prepare_q6k(w, row_bytes, rows, cols, img, s);
  if (ttype != TT_Q4_K) return hipErrorInvalidValue;
  const long nsb_total = (long)rows * (cols / 256);
  if (nsb_total <= 0) return hipSuccess;
  const unsigned grid = (unsigned)((nsb_total * 16 + 255) / 256);
  hipLaunchKernelGGL(k_mmq_prepare<TT_Q4_K>, dim3(grid), dim3(256), 0, s, (const uint8_t*)w, (uint8_t*)img,
                     nsb_total, row_bytes, cols / 256);
  return hipGetLastError();
}

// `ksplit` is already the launched slice count (mmq_slices); work holds
// mmq_split_bytes when it is above 1
template <int TT, int BT, int BR>
static hipError_t launch_mmq_img_t(const GemvArgs& g, int ksplit, void* work, hipStream_t s) {
  const int nsb = g.cols / 256;
  const long ntr = (g.rows + BR - 1) / BR, ntt = (g.tokens + BT - 1) / BT;
  const int cps = (nsb + ksplit - 1) / ksplit;
  const long G = ntr * ntt * ksplit;
  if (G > 0x7FFFFFFFL || (ksplit > 1 && ntr * ntt > kSkMaxTiles)) return hipErrorInvalidValue;
  unsigned* cnt = ksplit > 1 ? (unsigned*)work : nullptr;
  float* part = ksplit > 1 ? (float*)((uint8_t*)work + kSkCountBytes) : nullptr;
  hipLaunchKernelGGL((k_mmq_img<TT, BT, BR>), dim3((unsigned)G), dim3(256), 0, s, (const uint8_t*)g.w,
                     (const uint8_t*)g.xq, g.out, g.rows, g.tokens, nsb, g.act_bytes, (int)ntt, ksplit, cps, part,
                     cnt);
  return hipGetLastError();
}

template <int TT>
static hipError_t launch_mmq_img_type(const GemvArgs& g, int bt, int br, int ksplit, void* work, hipStream_t s) {
  if (bt == 64 && br == 64) return launch_mmq_img_t<TT, 64, 64>(g, ksplit, work, s);
  if (bt == 64 && br == 128) return launch_mmq_img_t<TT, 64, 128>(g, ksplit, work, s);
  if (bt == 128 && br == 64) return launch_mmq_img_t<TT, 128, 64>(g, ksplit, work, s);
  return hipErrorInvalidValue;
}

// Slices of the default image launch (small grids: split K over super-blocks,
// k_mmq's rule with one chunk = one super-block).
// One token tile: the small-grid rule (mmq_ksplit_for); several: whole rounds.
static int mmq_image_slices(const GemvArgs& g) {
  const int nsb = g.cols / 256;
  const long ntt = (g.tokens + 63) / 64;
  if (ntt >= 2) return mmq_slices(nsb, mmq_round_slices(ntt * ((g.rows + 63) / 64), nsb, 1));
  return mmq_slices(nsb, mmq_ksplit_for(g, 64, 64, nsb, 1));
}

long mmq_image_work_bytes(const GemvArgs& g) {
  if (g.ttype == TT_Q6_K) return bg_work_bytes(g, 0);
  return mmq_split_bytes(g, 64, 64, mmq_image_slices(g));
}

// g.w is the image; Q6_K: the plane-image MMQ, which has one shape (bt, br
// ignored)
hipError_t launch_mmq_image(const GemvArgs& g, int bt, int br, void* work, long work_bytes, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  if (g.ttype == TT_Q6_K) return launch_mmq_bg_q6k(g, work, work_bytes, s, 0);
  int ksplit = 1;
  if (bt <= 0 || br <= 0) {
    bt = 64;
    br = 64;
    ksplit = mmq_image_slices(g);
    if (!work || work_bytes < mmq_split_bytes(g, bt, br, ksplit)) ksplit = 1;
  }
  switch (g.ttype) {
    case TT_Q4_K: return launch_mmq_img_type<TT_Q4_K>(g, bt, br, ksplit, work, s);
    default: return hipErrorInvalidValue;
  }
}

// global_load_lds through inline assembly: the instruction the builtin emits
// (M0 = the wave's LDS destination; lane l's 16 / 4 bytes land at M0 + 16 l /
// 4 l), but invisible to the compiler's wait insertion, which otherwise makes
// every later LDS read of the same array wait for all copies in flight
// (vmcnt(0)) -- including the copy into the other stage just issued.  The
// caller orders the copies itself: each is issued before the loads that its
// later s_waitcnt vmcnt(N) leaves in flight (vector memory loads complete in
// issue order), and a barrier follows that wait.  The compiler's own vmcnt
// waits stay sufficient with these extra loads in the queue: it counts fewer
// newer loads than there are, so it waits longer, never shorter.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}
// (M0 is saved and restored around the copy: the compiler keeps it reserved.)
__device__ __forceinline__ void lds_copy16(const void* src, const void* lds_dst) {
  uint32_t keep;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
      : "=&s"(keep)
      : "v"(src), "s"(lds_addr(lds_dst))
      : "memory");
}
__device__ __forceinline__ void lds_copy4(const void* src, const void* lds_dst) {
  uint32_t keep;
  asm volatile(
      "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
      : "=&s"(keep)
      : "v"(src), "s"(lds_addr(lds_dst))
      : "memory");
}

// ---- weights-direct MMQ (Q4_K, 32 or 64 tokens x 128 rows) -----------------------------------
// Each wave owns 32 weight rows and reads their Q4_K bytes from global memory
// straight into MFMA B fragments, with no LDS image of the weights: lane l
// holds row l%32, and each 16-byte qs piece gives it values 16*(l/32)..+15 of
// two sub-blocks (low / high nibbles), scaled by the split sub-block scale as
// in k_mmq.  The workgroup's BT = 32 NA tokens of Q8_K activation are copied
// into LDS by global_load_lds (DMA, no registers), double-buffered: chunk c+1
// (one super-block) lands while chunk c is multiplied.  LDS token row:
// qs[256] | bsums[16] | d, 304 bytes, so 16-byte fragment reads of 32
// consecutive tokens fall 12 banks apart (conflict-free).  K may be cut into
// ksplit slices of cps super-blocks (small grids: few tokens), the partial
// tiles added in slice order by the tile's last workgroup (mmq_write_tile).
// The copies are issued as inline assembly (lds_copy16), so the super-block's
// LDS reads do not wait for the copy into the other stage (config 5 Q4_K from
// the fragment image, two weight copies rotated: unsplit T = 64 / 512 33.6 /
// 127.3 us against 41.2 / 136.3 with the builtin's copies; with the mirror's
// K split T = 32 / 64 / 128 18.6 / 28.4 / 40.8 against 19.4 / 29.8 / 43.3).
// Measured on MI355X, config
// 5 Q4_K [17408, 5120]: T = 512 146-150 us (before the fragment image)
// against 184 us for the 64 x 64 tile kernel in the same harness, T = 128 56
// against 62 us; with the split, T = 8 / 16 / 32 / 64 20.3 / 20.8 / 21.6 /
// 32.3 us against 24.1 / 24.1 / 24.2 / 32.5 for the tile kernel's split
// launch.
constexpr int kWdRow = 304, kWdPieces = 19, kWdBR = 128;

// Q4_K fragment image: the GGUF bytes permuted, the same 144 bytes per row and
// super-block.  Rows in groups of 32 (the last group padded with zero rows);
// group r, super-block sb is a 4608-byte tile at (r * nsb + sb) * 4608:
//   [0, 4096)     lane L = i + 32 k (row i of the group, half k) holds the qs
//                 bytes 32c + 16k .. +15 of row i at 1024 c + 16 L (c < 4)
//   [4096, 4608)  row i's 16-byte header (d, dmin, the 12 scale bytes) at
//                 4096 + 16 i
// so each wave instruction of the weights-direct kernels loads one aligned,
// contiguous 1 KB (512 bytes for the headers) instead of 32 rows' pieces.
constexpr int kWdiTile4 = 4608;

// Makes the loaded registers complete here: the compiler may otherwise sink
// the prologue's weight loads past the barrier into the loop, where the wait
// for them then stalls every iteration on the loads in flight for the next.
template <class T>
__device__ __forceinline__ T wd_pinned(T v) {
  asm volatile("" : "+v"(v));
  return v;
}
#define wd_pin(x) ((x) = wd_pinned(x))

__device__ __forceinline__ uint32_t pk_mul_u16(uint32_t v, u16x2 m) {
  return __builtin_bit_cast(uint32_t, (u16x2)(__builtin_bit_cast(u16x2, v) * m));
}

// Grid of a weights-direct launch: workgroups [0, nwhole) take whole tiles
// 0 .. nwhole - 1 (all of K); the rest take the remaining tiles cut into
// ksplit slices of cps super-blocks.  nwhole = 0 splits every tile; ksplit = 1
// splits none.  The sliced tiles come last in the grid, so they fill the
// final, partial round of resident workgroups instead of leaving it to a few.
// Within each part, block b's tile is XCD-contiguous (b % 8 is the XCD the
// block is dispatched to), and the slices are ordered (group of ntile_t
// tiles, slice, tile): the workgroups side by side read the same weights at
// the same K (Q4_K config 5 at 256 / 512 tokens 72.9 / 130.4 us against
// 77.5 / 133.6 slice-minor, every tile split).  Sets the tile, its slice and
// the slice count of this workgroup, and the index of its partial tiles among
// the sliced ones.
struct WdTile {
  int tile, ks, ksplit, su;
};
__device__ __forceinline__ WdTile wd_tile(int ntile_t, int nwhole, int ksplit) {
  const int G = gridDim.x, b = blockIdx.x;
  WdTile r;
  if (b < nwhole || ksplit <= 1) {
    const int n = ksplit <= 1 ? G : nwhole;
    r.tile = (n & 7) == 0 ? (b & 7) * (n >> 3) + (b >> 3) : b;
    r.ks = 0;
    r.ksplit = 1;
    r.su = 0;
    return r;
  }
  const int np = G - nwhole, nsplit = np / ksplit;
  int p = b - nwhole;
  if ((np & 7) == 0) p = (p & 7) * (np >> 3) + (p >> 3);
  const int gw = ntile_t < nsplit ? ntile_t : nsplit, full = nsplit / gw, rem = nsplit - full * gw;
  if (p < full * ksplit * gw) {
    const int grp = p / (ksplit * gw), loc = p - grp * ksplit * gw;
    r.ks = loc / gw;
    r.su = grp * gw + (loc - r.ks * gw);
  } else {
    const int loc = p - full * ksplit * gw;
    r.ks = loc / rem;
    r.su = full * gw + (loc - r.ks * rem);
  }
  r.tile = nwhole + r.su;
  r.ksplit = ksplit;
  return r;
}

template <int NA, bool IMG>
__global__ __launch_bounds__(256) void k_mmq_wd_q4k(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ,
                                                     float* __restrict__ Y, int rows, int tokens, long row_bytes,
                                                     long act_bytes, int nsb, int ntile_t, int nwhole, int ksplit,
                                                     int cps, float* __restrict__ part, unsigned* __restrict__ cnt) {
  constexpr int BT = 32 * NA, STAGE = BT * kWdRow, NDMA = (BT * kWdPieces + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint8_t act[2][STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 31, lh = lane >> 5;
  const WdTile wt = wd_tile(ntile_t, nwhole, ksplit);
  const int rt = wt.tile / ntile_t, tt = wt.tile - rt * ntile_t, ks = wt.ks;
  const int r0 = rt * kWdBR, t0 = tt * BT;
  const uint8_t* wrow;
  if constexpr (IMG) {
    // this wave's group of 32 rows (a group past the end re-reads the last)
    const int ngrp = (rows + 31) >> 5, grp = (r0 >> 5) + wv;
    wrow = W + (long)(grp < ngrp ? grp : ngrp - 1) * nsb * kWdiTile4;
  } else {
    const int row = r0 + 32 * wv + li;
    wrow = W + (long)(row < rows ? row : rows - 1) * row_bytes;
  }
  const int sb0 = wt.ksplit > 1 ? ks * cps : 0;
  const int sb1 = wt.ksplit > 1 && sb0 + cps < nsb ? sb0 + cps : nsb;

  // DMA piece p = 64*(4i + wave) + lane of the stage: token p/19, 16-byte
  // slot p%19 (16 qs slots, two bsum slots, one slot holding d); tokens past
  // the end re-read the last one
  long goff[NDMA];
  bool gon[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int p = 64 * (4 * i + wv) + lane;
    gon[i] = p < BT * kWdPieces;
    const int tp = p / kWdPieces, j = p - tp * kWdPieces;
    int tok = t0 + tp;
    tok = tok < tokens ? tok : tokens - 1;
    goff[i] = (long)tok * act_bytes + (j < 16 ? 4 + 16 * j : j == 16 ? 260 : j == 17 ? 276 : 0);
  }
  auto issue_act = [&](int sb, uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      if (4 * i + wv < (BT * kWdPieces + 63) / 64 && gon[i])
        lds_copy16(XQ + goff[i] + 292L * sb, buf + 1024 * (4 * i + wv));
    }
  };
  u32x4 wh, wq[4];
  auto issue_w = [&](int sb, u32x4& h, u32x4 (&q)[4]) {
    if constexpr (IMG) {
      const uint8_t* b = wrow + (long)kWdiTile4 * sb;
      h = *(const u32x4*)(b + 4096 + 16 * li);
#pragma unroll
      for (int c = 0; c < 4; ++c) q[c] = *(const u32x4*)(b + 1024 * c + 16 * lane);
    } else {
      const uint8_t* b = wrow + 144L * sb;
      h = *(const u32x4*)b;
#pragma unroll
      for (int c = 0; c < 4; ++c) q[c] = *(const u32x4*)(b + 16 + 32 * c + 16 * lh);
    }
  };

  f32x16 acc[NA][1];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[a][0][e] = 0.0f;
  const i32x16 zero = {};
  const f32x16 fz = {};

  issue_act(sb0, &act[0][0]);
  issue_w(sb0, wh, wq);
  wd_pin(wh);
#pragma unroll
  for (int c = 0; c < 4; ++c) wd_pin(wq[c]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // one super-block: compute from A while super-block sb + 1 lands in nxt
  for (int sb = sb0; sb < sb1; ++sb) {
    const int cur = (sb - sb0) & 1;
    const uint8_t* A = &act[cur][0];
    uint8_t* nxt = &act[cur ^ 1][0];
    u32x4 nh, nq[4];
    if (sb + 1 < sb1) {
      issue_act(sb + 1, nxt);
      issue_w(sb + 1, nh, nq);
    }
    __builtin_amdgcn_iglp_opt(0);
    // 6-bit scales and mins of this lane's row (kernels256.c:105-125)
    const uint32_t S0 = wh.y, S1 = wh.z, S2 = wh.w;
    const uint32_t sc_lo = S0 & 0x3F3F3F3Fu, mn_lo = S1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u);
    i32x16 chi[NA], clo[NA];
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      chi[a] = zero;
      clo[a] = zero;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint32_t q0 = wq[c].x, q1 = wq[c].y, q2 = wq[c].z, q3 = wq[c].w;
#pragma unroll
      for (int hi = 0; hi < 2; ++hi) {
        const int s = 2 * c + hi;
        const uint32_t n0 = (hi ? q0 >> 4 : q0) & 0x0F0F0F0Fu, n1 = (hi ? q1 >> 4 : q1) & 0x0F0F0F0Fu;
        const uint32_t n2 = (hi ? q2 >> 4 : q2) & 0x0F0F0F0Fu, n3 = (hi ? q3 >> 4 : q3) & 0x0F0F0F0Fu;
        const uint32_t sc = ((s < 4 ? sc_lo : sc_hi) >> (8 * (s & 3))) & 63u;
        const u16x2 mh = {(uint16_t)(sc >> 3), (uint16_t)(sc >> 3)};
        const u16x2 ml = {(uint16_t)(sc & 7u), (uint16_t)(sc & 7u)};
        const i32x4 bh = {(int)pk_mul_u16(n0, mh), (int)pk_mul_u16(n1, mh), (int)pk_mul_u16(n2, mh),
                          (int)pk_mul_u16(n3, mh)};
        const i32x4 bl = {(int)pk_mul_u16(n0, ml), (int)pk_mul_u16(n1, ml), (int)pk_mul_u16(n2, ml),
                          (int)pk_mul_u16(n3, ml)};
#pragma unroll
        for (int a = 0; a < NA; ++a) {
          const i32x4 af = *(const i32x4*)(A + (32 * a + li) * kWdRow + 32 * s + 16 * lh);
          chi[a] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bh, chi[a], 0, 0, 0);
          clo[a] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bl, clo[a], 0, 0, 0);
        }
      }
    }
    // mins: summs[t][r] = sum_j bsum[t][j] * min[r][j/2], exact in the f16 MFMA
    const uint32_t mn = lh ? mn_hi : mn_lo;
    f16x8 bm;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const _Float16 m = (_Float16)(float)((mn >> (8 * k)) & 255u);
      bm[2 * k] = m;
      bm[2 * k + 1] = m;
    }
    const float d = h2f(wh.x), ndm = -h2f(wh.x >> 16);
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      const i16x8 bs = *(const i16x8*)(A + (32 * a + li) * kWdRow + 256 + 16 * lh);
      f16x8 am;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const short v = bs[k];
        am[k] = (_Float16)v;
      }
      const f32x16 cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, fz, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int t = 32 * a + 8 * (e >> 2) + 4 * lh + (e & 3);
        const float dy = *(const float*)(A + t * kWdRow + 288);
        const int ci = chi[a][e], cl = clo[a][e];  // (scalar copies: see k_mmq)
        const int isum = 8 * ci + cl;
        const float inner = __builtin_fmaf(d, (float)isum, ndm * cm[e]);
        acc[a][0][e] = __builtin_fmaf(dy, inner, acc[a][0][e]);
      }
    }
    // the whole super-block's products and epilogue stay above the wait:
    // otherwise the scheduler may sink half of them below it, so the loads
    // for sb + 1 get only the first half to land in
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0);  // chunk sb+1: DMA and weight registers
    __syncthreads();
    if (sb + 1 < sb1) {
      wh = nh;
#pragma unroll
      for (int c = 0; c < 4; ++c) wq[c] = nq[c];
    }
  }
  mmq_write_tile<NA, 1, 4>(acc, Y, rows, tokens, r0, t0, 32 * wv, 0, wt.su, wt.ksplit, ks, part, cnt);
}

// Few tokens (T <= 8 NG, NG < 4; one 32-token tile): the same staging, one
// MFMA per sub-block on the raw nibbles, and the sub-block scale applied to
// the integer result by an integer multiply-add (isum = sum_j sc_j S_j,
// kernels256.c:474-498) -- but only on the accumulator elements of real
// tokens: lane element e holds token 8 (e / 4) + 4 (lane / 32) + e % 4, so the
// first 4 NG elements cover tokens 0 .. 8 NG - 1.  The split-scale planes of
// k_mmq_wd_q4k cost two products per weight value and two MFMAs whatever the
// token count; here the per-weight work is the nibble extraction alone.
// One super-block of k_mmq_wds_q4k / k_mmq_rk: one MFMA per 32-value
// sub-block on the raw nibbles, the sub-block scale applied to the integer
// result on the NE kept elements, the mins through an exact f16 MFMA, then
// acc[0][0] += dy * (d * isum - dmin * summs).  A macro, as the Q6_K one.
#define QHIP_Q4K_SUPERBLOCK(wh_, wq_, A, arow)                                                                       \
  do {                                                                                                               \
    const i32x16 zero_ = {};                                                                                         \
    const f32x16 fz_ = {};                                                                                           \
    const uint32_t S0_ = (wh_).y, S1_ = (wh_).z, S2_ = (wh_).w;                                                      \
    const uint32_t sc_lo_ = S0_ & 0x3F3F3F3Fu, mn_lo_ = S1_ & 0x3F3F3F3Fu;                                           \
    const uint32_t sc_hi_ = (S2_ & 0x0F0F0F0Fu) | ((S0_ >> 2) & 0x30303030u);                                        \
    const uint32_t mn_hi_ = ((S2_ >> 4) & 0x0F0F0F0Fu) | ((S1_ >> 2) & 0x30303030u);                                 \
    int isum_[NE];                                                                                                   \
    _Pragma("unroll") for (int e_ = 0; e_ < NE; ++e_) isum_[e_] = 0;                                                 \
    _Pragma("unroll") for (int c_ = 0; c_ < 4; ++c_) {                                                               \
      const uint32_t q0_ = (wq_)[c_].x, q1_ = (wq_)[c_].y, q2_ = (wq_)[c_].z, q3_ = (wq_)[c_].w;                     \
      _Pragma("unroll") for (int hi_ = 0; hi_ < 2; ++hi_) {                                                          \
        const int s_ = 2 * c_ + hi_;                                                                                 \
        const i32x4 bq_ = {(int)((hi_ ? q0_ >> 4 : q0_) & 0x0F0F0F0Fu), (int)((hi_ ? q1_ >> 4 : q1_) & 0x0F0F0F0Fu), \
                          (int)((hi_ ? q2_ >> 4 : q2_) & 0x0F0F0F0Fu), (int)((hi_ ? q3_ >> 4 : q3_) & 0x0F0F0F0Fu)}; \
        const int sc_ = (int)(((s_ < 4 ? sc_lo_ : sc_hi_) >> (8 * (s_ & 3))) & 63u);                                 \
        const i32x4 af_ = *(const i32x4*)((A) + (arow) * kWdRow + 32 * s_ + 16 * lh);                                \
        const i32x16 S_ = __builtin_amdgcn_mfma_i32_32x32x32_i8(af_, bq_, zero_, 0, 0, 0);                           \
        _Pragma("unroll") for (int e_ = 0; e_ < NE; ++e_) isum_[e_] += sc_ * S_[e_];                                 \
      }                                                                                                              \
    }                                                                                                                \
    /* mins: summs[t][r] = sum_j bsum[t][j] * min[r][j/2], exact in the f16 MFMA */                                  \
    const uint32_t mn_ = lh ? mn_hi_ : mn_lo_;                                                                       \
    f16x8 bm_;                                                                                                       \
    _Pragma("unroll") for (int k_ = 0; k_ < 4; ++k_) {                                                               \
      const _Float16 m_ = (_Float16)(float)((mn_ >> (8 * k_)) & 255u);                                               \
      bm_[2 * k_] = m_;                                                                                              \
      bm_[2 * k_ + 1] = m_;                                                                                          \
    }                                                                                                                \
    const float d_ = h2f((wh_).x), ndm_ = -h2f((wh_).x >> 16);                                                       \
    const i16x8 bs_ = *(const i16x8*)((A) + (arow) * kWdRow + 256 + 16 * lh);                                        \
    f16x8 am_;                                                                                                       \
    _Pragma("unroll") for (int k_ = 0; k_ < 8; ++k_) {                                                               \
      const short v_ = bs_[k_];                                                                                      \
      am_[k_] = (_Float16)v_;                                                                                        \
    }                                                                                                                \
    const f32x16 cm_ = __builtin_amdgcn_mfma_f32_32x32x16_f16(am_, bm_, fz_, 0, 0, 0);                               \
    _Pragma("unroll") for (int e_ = 0; e_ < NE; ++e_) {                                                              \
      const int t_ = 8 * (e_ >> 2) + 4 * lh + (e_ & 3);                                                              \
      const float dy_ = *(const float*)((A) + t_ * kWdRow + 288);                                                    \
      const float inner_ = __builtin_fmaf(d_, (float)isum_[e_], ndm_ * cm_[e_]);                                     \
      acc[0][0][e_] = __builtin_fmaf(dy_, inner_, acc[0][0][e_]);                                                    \
    }                                                                                                                \
  } while (0)

template <int NG>
__global__ __launch_bounds__(256) void k_mmq_wds_q4k(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ,
                                                      float* __restrict__ Y, int rows, int tokens, long row_bytes,
                                                      long act_bytes, int nsb, int ksplit, int cps,
                                                      float* __restrict__ part, unsigned* __restrict__ cnt) {
  constexpr int BT = 32, STAGE = BT * kWdRow, NDMA = (BT * kWdPieces + 255) / 256, NE = 4 * NG;
  __shared__ __attribute__((aligned(16))) uint8_t act[2][STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 31, lh = lane >> 5;
  const int G = gridDim.x;
  int g = blockIdx.x;
  if ((G & 7) == 0) g = (g & 7) * (G >> 3) + (g >> 3);  // XCD-contiguous tiles, as k_mmq
  const int ks = g % ksplit;
  g /= ksplit;
  const int r0 = g * kWdBR;
  const int row = r0 + 32 * wv + li;
  const uint8_t* wrow = W + (long)(row < rows ? row : rows - 1) * row_bytes;
  const int sb0 = ks * cps, sb1 = sb0 + cps < nsb ? sb0 + cps : nsb;

  long goff[NDMA];
  bool gon[NDMA];
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int p = 64 * (4 * i + wv) + lane;
    gon[i] = p < BT * kWdPieces;
    const int tp = p / kWdPieces, j = p - tp * kWdPieces;
    const int tok = tp < tokens ? tp : tokens - 1;
    goff[i] = (long)tok * act_bytes + (j < 16 ? 4 + 16 * j : j == 16 ? 260 : j == 17 ? 276 : 0);
  }
  auto issue_act = [&](int sb, uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      if (4 * i + wv < (BT * kWdPieces + 63) / 64 && gon[i])
        lds_copy16(XQ + goff[i] + 292L * sb, buf + 1024 * (4 * i + wv));
    }
  };
  u32x4 wh, wq[4];
  auto issue_w = [&](int sb, u32x4& h, u32x4 (&q)[4]) {
    const uint8_t* b = wrow + 144L * sb;
    h = *(const u32x4*)b;
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = *(const u32x4*)(b + 16 + 32 * c + 16 * lh);
  };

  f32x16 acc[1][1];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[0][0][e] = 0.0f;

  issue_act(sb0, &act[0][0]);
  issue_w(sb0, wh, wq);
  wd_pin(wh);
#pragma unroll
  for (int c = 0; c < 4; ++c) wd_pin(wq[c]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  // one super-block: compute from A while super-block sb + 1 lands in nxt
  for (int sb = sb0; sb < sb1; ++sb) {
    const int cur = (sb - sb0) & 1;
    const uint8_t* A = &act[cur][0];
    uint8_t* nxt = &act[cur ^ 1][0];
    u32x4 nh, nq[4];
    if (sb + 1 < sb1) {
      issue_act(sb + 1, nxt);
      issue_w(sb + 1, nh, nq);
    }
    QHIP_Q4K_SUPERBLOCK(wh, wq, A, li);
    __builtin_amdgcn_s_waitcnt(0);  // chunk sb+1: DMA and weight registers
    __syncthreads();
    if (sb + 1 < sb1) {
      wh = nh;
#pragma unroll
      for (int c = 0; c < 4; ++c) wq[c] = nq[c];
    }
  }
  mmq_write_tile<1, 1, 4, NE>(acc, Y, rows, tokens, r0, 0, 32 * wv, 0, g, ksplit, ks, part, cnt);
}

// Q6_K, few tokens (T <= 8 NG; one 32-token tile): the weights-direct
// structure of k_mmq_wds_q4k on the Q6_K bytes.  Lane l of a wave holds row
// l%32 and, for 16-value group g = 8h + m + 2q (kernels256.c:720-738, values
// 128h + 32q + 16m + 0..15), its values 8(l/32)..+7: bytes of ql at 64h +
// 32(q&1) + 16m + 8(l/32) (low nibble for q < 2, high for q >= 2) and the
// 2-bit field 2q of qh at 32h + 16m + 8(l/32), decoded as the unsigned 6-bit
// value u = q6.  One v_mfma_i32_32x32x16_i8 per group gives S_g = sum u*q8;
// the reference's integer isum = sum_g sc_g sum (u - 32) q8 = sum_g sc_g S_g
// - 32 sum_g sc_g bsum_g, the last sum by an exact f16 MFMA (bsums below 2048,
// scales int8, every partial sum below 2^24).  Scaling and epilogue only on
// the accumulator elements of real tokens.
//
// IMG = false reads the GGUF rows (NG < 4): 14 loads per lane and super-block,
// most of them misaligned (210-byte blocks) and each spanning 32 rows -- the
// texture path, not HBM, bounds it.  IMG = true reads the fragment image
// below: 8 loads per lane, each wave instruction one aligned, contiguous 1 KB.
//
// Q6_K fragment image: the GGUF bytes permuted, the same 210 bytes per row and
// super-block.  Rows in groups of 32 (the last group padded with zero rows);
// group r, super-block sb is a 6720-byte tile at (r * nsb + sb) * 6720:
//   [0, 6144)     lane L = i + 32 k (row i of the group, value half k) holds 24
//                 dwords, piece c = dwords 4c..4c+3 at 1024 c + 16 L; dwords
//                 6j..6j+5 for j = 2h + m are the 8 bytes of ql at 64h + 16m +
//                 8k, of ql at 64h + 32 + 16m + 8k, and of qh at 128 + 32h +
//                 16m + 8k
//   [6144, 6656)  row i's 16 int8 scales at 6144 + 16 i
//   [6656, 6720)  row i's f16 d at 6656 + 2 i
constexpr int kWdiTile = 6720;

template <bool IMG>
struct Q6Regs;
template <>
struct Q6Regs<false> {
  u32x2 la[4], lb[4], qh[4];
  u32x4 sc;
  uint32_t d;
  __device__ __forceinline__ uint32_t ql(int j, int odd, int k) const { return odd ? lb[j][k] : la[j][k]; }
  __device__ __forceinline__ uint32_t qhi(int j, int k) const { return qh[j][k]; }
  __device__ __forceinline__ void pin() {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wd_pin(la[j]);
      wd_pin(lb[j]);
      wd_pin(qh[j]);
    }
    wd_pin(sc);
    wd_pin(d);
  }
};
template <>
struct Q6Regs<true> {
  u32x4 p[6];
  u32x4 sc;
  uint32_t d;
  __device__ __forceinline__ uint32_t at(int i) const { return p[i >> 2][i & 3]; }
  __device__ __forceinline__ uint32_t ql(int j, int odd, int k) const { return at(6 * j + 2 * odd + k); }
  __device__ __forceinline__ uint32_t qhi(int j, int k) const { return at(6 * j + 4 + k); }
  __device__ __forceinline__ void pin() {
#pragma unroll
    for (int c = 0; c < 6; ++c) wd_pin(p[c]);
    wd_pin(sc);
    wd_pin(d);
  }
};

// One super-block of k_mmq_wds_q6k / k_mmq_wdp_q6k / k_mmq_rk: the 16 group MFMAs on
// this lane's decoded 6-bit values (B, from the Q6Regs `wc`) against the
// staged activation row `arow` of `A`, the integer scaling and the -32
// offset on the NE kept elements, then acc[0][0] += dy * d * isum.  A macro,
// not a function: the same code behind a call boundary (even forced inline)
// is scheduled with 13-93 more VGPRs by this compiler.
#define QHIP_Q6K_SUPERBLOCK(wc, A, arow)                                                   \
  do {                                                                                     \
    const i32x16 zero_ = {};                                                               \
    const f32x16 fz_ = {};                                                                 \
    const uint32_t scw_[4] = {(wc).sc.x, (wc).sc.y, (wc).sc.z, (wc).sc.w};                 \
    int isum_[NE];                                                                         \
    _Pragma("unroll") for (int e_ = 0; e_ < NE; ++e_) isum_[e_] = 0;                       \
    _Pragma("unroll") for (int j_ = 0; j_ < 4; ++j_) {                                     \
      const int h_ = j_ >> 1, m_ = j_ & 1;                                                 \
      _Pragma("unroll") for (int q_ = 0; q_ < 4; ++q_) {                                   \
        const int grp_ = 8 * h_ + m_ + 2 * q_;                                             \
        uint32_t v_[2];                                                                    \
        _Pragma("unroll") for (int k_ = 0; k_ < 2; ++k_) {                                 \
          const uint32_t l_ = (wc).ql(j_, q_ & 1, k_), x_ = (wc).qhi(j_, k_);              \
          const uint32_t nib_ = (q_ >= 2 ? l_ >> 4 : l_) & 0x0F0F0F0Fu;                    \
          const uint32_t hi_ = q_ == 0 ? (x_ << 4) & 0x30303030u                           \
                              : q_ == 1 ? (x_ << 2) & 0x30303030u                          \
                              : q_ == 2 ? x_ & 0x30303030u                                 \
                                       : (x_ >> 2) & 0x30303030u;                          \
          v_[k_] = nib_ | hi_;                                                             \
        }                                                                                  \
        const long bq_ = (long)(((unsigned long)v_[1] << 32) | v_[0]);                     \
        const long af_ = *(const long*)((A) + (arow) * kWdRow + 16 * grp_ + 8 * lh);       \
        const i32x16 S_ = __builtin_amdgcn_mfma_i32_32x32x16_i8(af_, bq_, zero_, 0, 0, 0); \
        const int sc_ = (int)(int8_t)(scw_[grp_ >> 2] >> (8 * (grp_ & 3)));                \
        _Pragma("unroll") for (int e_ = 0; e_ < NE; ++e_) isum_[e_] += sc_ * S_[e_];       \
      }                                                                                    \
    }                                                                                      \
    /* sum_g sc_g bsum_g[t], exact in the f16 MFMA: A = the token's 8 bsums of              \
       groups 8(l/32)..+7, B = the row's scales of the same groups */                       \
    const i16x8 bs_ = *(const i16x8*)((A) + (arow) * kWdRow + 256 + 16 * lh);              \
    f16x8 am_, bm_;                                                                         \
    _Pragma("unroll") for (int k_ = 0; k_ < 8; ++k_) {                                     \
      const short bv_ = bs_[k_];                                                           \
      am_[k_] = (_Float16)bv_;                                                             \
      bm_[k_] = (_Float16)(float)(int)(int8_t)(scw_[2 * lh + (k_ >> 2)] >> (8 * (k_ & 3))); \
    }                                                                                      \
    const f32x16 cm_ = __builtin_amdgcn_mfma_f32_32x32x16_f16(am_, bm_, fz_, 0, 0, 0);      \
    const float dw_ = h2f((wc).d);                                                         \
    /* the reference's integer (kernels256.c:720-738) */                                   \
    _Pragma("unroll") for (int e_ = 0; e_ < NE; ++e_) {                                    \
      const int t_ = 8 * (e_ >> 2) + 4 * lh + (e_ & 3);                                    \
      const float dy_ = *(const float*)((A) + t_ * kWdRow + 288);                          \
      const int tot_ = isum_[e_] - 32 * (int)cm_[e_];                                      \
      acc[0][0][e_] = __builtin_fmaf(dy_, dw_ * (float)tot_, acc[0][0][e_]);               \
    }                                                                                      \
  } while (0)

// DMA offsets of the activation pieces a lane moves: piece P = 64 (4i + wave)
// + lane of a run of stages of TR token rows: stage P / (19 TR), token row
// (P % (19 TR)) / 19, 16-byte slot (P % (19 TR)) % 19 (16 qs slots, two bsum
// slots, one holding d); rows past the last token re-read it.  st[i] = the
// piece's stage, or nst when the piece is past the run.
template <int NDMA, int TR>
__device__ __forceinline__ void wd_dma_plan(int wv, int lane, int tokens, long act_bytes, int nst, long (&off)[NDMA],
                                            int (&st)[NDMA]) {
  constexpr int NPC = TR * kWdPieces;
#pragma unroll
  for (int i = 0; i < NDMA; ++i) {
    const int P = 64 * (4 * i + wv) + lane;
    const int sg = P / NPC, p = P - sg * NPC;
    const int tp = p / kWdPieces, j = p - tp * kWdPieces;
    const int tok = tp < tokens ? tp : tokens - 1;
    st[i] = P < nst * NPC ? sg : nst;
    off[i] = (long)tok * act_bytes + (j < 16 ? 4 + 16 * j : j == 16 ? 260 : j == 17 ? 276 : 0);
  }
}

// GGUF rows, T <= 8 NG (NG < 4), two stages double-buffered: super-block sb + 1
// is loaded while sb is multiplied.  Only the 8 NG token rows the kept
// elements read are staged (lanes of later rows read row 0: their MFMA
// columns are never kept).
template <int NG>
__global__ __launch_bounds__(256) void k_mmq_wds_q6k(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ,
                                                      float* __restrict__ Y, int rows, int tokens, long row_bytes,
                                                      long act_bytes, int nsb, int ksplit, int cps,
                                                      float* __restrict__ part, unsigned* __restrict__ cnt) {
  constexpr int TR = 8 * NG, NE = 4 * NG, STAGE = TR * kWdRow, NPC = TR * kWdPieces, NDMA = (NPC + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint8_t act[2][STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 31, lh = lane >> 5;
  const int G = gridDim.x;
  int g = blockIdx.x;
  if ((G & 7) == 0) g = (g & 7) * (G >> 3) + (g >> 3);  // XCD-contiguous tiles, as k_mmq
  const int ks = g % ksplit;
  g /= ksplit;
  const int r0 = g * kWdBR;
  const int row = r0 + 32 * wv + li;
  const uint8_t* wrow = W + (long)(row < rows ? row : rows - 1) * row_bytes;
  const int sb0 = ks * cps, sb1 = sb0 + cps < nsb ? sb0 + cps : nsb;
  const int arow = li < TR ? li : 0;

  long goff[NDMA];
  int gst[NDMA];
  wd_dma_plan<NDMA, TR>(wv, lane, tokens, act_bytes, 1, goff, gst);
  auto issue_act = [&](int sb, uint8_t* buf) {
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      if (4 * i + wv < (NPC + 63) / 64 && gst[i] == 0)
        lds_copy16(XQ + goff[i] + 292L * sb, buf + 1024 * (4 * i + wv));
    }
  };
  auto issue_w = [&](int sb, Q6Regs<false>& q) {
    const uint8_t* b = wrow + 210L * sb;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int h = j >> 1, m = j & 1;
      q.la[j] = *(const u32x2_u*)(b + 64 * h + 16 * m + 8 * lh);
      q.lb[j] = *(const u32x2_u*)(b + 64 * h + 32 + 16 * m + 8 * lh);
      q.qh[j] = *(const u32x2_u*)(b + 128 + 32 * h + 16 * m + 8 * lh);
    }
    q.sc = *(const u32x4_u*)(b + 192);
    q.d = *(const uint16_t*)(b + 208);
  };

  f32x16 acc[1][1];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[0][0][e] = 0.0f;

  Q6Regs<false> wc, wn;
  issue_act(sb0, &act[0][0]);
  issue_w(sb0, wc);
  wc.pin();
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int sb = sb0; sb < sb1; ++sb) {
    const int cur = (sb - sb0) & 1;
    if (sb + 1 < sb1) {
      issue_act(sb + 1, &act[cur ^ 1][0]);
      issue_w(sb + 1, wn);
    }
    QHIP_Q6K_SUPERBLOCK(wc, &act[cur][0], arow);
    __builtin_amdgcn_s_waitcnt(0);  // chunk sb+1: DMA and weight registers
    __syncthreads();
    if (sb + 1 < sb1) wc = wn;
  }
  mmq_write_tile<1, 1, 4, NE>(acc, Y, rows, tokens, r0, 0, 32 * wv, 0, g, ksplit, ks, part, cnt);
}

// The fragment image, T <= 8 NG per token tile (blockIdx.y; 33..64 tokens
// two tiles of 32): the workgroup's K slice in groups of CPS super-blocks,
// each group's weight loads (8 per lane and super-block, every wave
// instruction one aligned 1 KB) and activation DMA all issued before any of
// it is used.  Measured on MI355X, config 5 Q6_K [5120, 17408], 1 / 8 / 16 /
// 24 tokens: 21.1 / 21.4 / 24.1 / 28.0 us with CPS = 2, against 22.1 / 22.2
// / 24.4 / 28.2 double-buffered one super-block at a time and 22.5 / 22.7 /
// 25.9 / 30.4 with CPS = 3 (more registers, fewer resident workgroups).  The
// two token tiles of a row tile run side by side and share its weight reads
// in L2: 40 / 48 / 64 tokens 47.7 / 46.8 / 46.9 us with the K split planned
// over both tiles' workgroups (54 us with one tile's split), against 49.0 /
// 49.4 / 49.1 from the plane image; [2560, 9728] 21.1 / 21.4 at 48 / 64
// against 21.8 / 21.9.
template <int NG, int CPS>
__global__ __launch_bounds__(256) void k_mmq_wdp_q6k(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ,
                                                      float* __restrict__ Y, int rows, int tokens, long act_bytes,
                                                      int nsb, int ksplit, int cps, float* __restrict__ part,
                                                      unsigned* __restrict__ cnt) {
  constexpr int TR = 8 * NG, NE = 4 * NG;
  constexpr int STAGE = TR * kWdRow, NPC = TR * kWdPieces, NDMA = (CPS * NPC + 255) / 256;
  __shared__ __attribute__((aligned(16))) uint8_t act[CPS * STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 31, lh = lane >> 5;
  const int G = gridDim.x;
  int g = blockIdx.x;
  if ((G & 7) == 0) g = (g & 7) * (G >> 3) + (g >> 3);  // XCD-contiguous tiles, as k_mmq
  const int ks = g % ksplit;
  g /= ksplit;
  const int r0 = g * kWdBR;
  // this wave's group of 32 rows (a group past the end re-reads the last)
  const int ngrp = (rows + 31) >> 5, grp = (r0 >> 5) + wv;
  const uint8_t* wbase = W + (long)(grp < ngrp ? grp : ngrp - 1) * nsb * kWdiTile;
  const int sb0 = ks * cps, sb1 = sb0 + cps < nsb ? sb0 + cps : nsb;
  const int arow = li < TR ? li : 0;
  // token tile blockIdx.y (T > 32: NG = 4): its tokens' activation rows and
  // outputs; its row tiles' split-K hand-offs follow those of tile y - 1
  XQ += (long)blockIdx.y * TR * act_bytes;
  Y += (long)blockIdx.y * TR * rows;
  tokens = tokens - (int)blockIdx.y * TR < TR ? tokens - (int)blockIdx.y * TR : TR;
  const int tile = g + (int)blockIdx.y * (G / ksplit);

  long goff[NDMA];
  int gst[NDMA];
  wd_dma_plan<NDMA, TR>(wv, lane, tokens, act_bytes, CPS, goff, gst);

  f32x16 acc[1][1];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[0][0][e] = 0.0f;

  for (int base = sb0; base < sb1; base += CPS) {
    const int n = sb1 - base < CPS ? sb1 - base : CPS;
    Q6Regs<true> wr[CPS];
#pragma unroll
    for (int s = 0; s < CPS; ++s) {
      if (s < n) {
        const uint8_t* b = wbase + (long)kWdiTile * (base + s);
#pragma unroll
        for (int c = 0; c < 6; ++c) wr[s].p[c] = *(const u32x4*)(b + 1024 * c + 16 * lane);
        wr[s].sc = *(const u32x4*)(b + 6144 + 16 * li);
        wr[s].d = *(const uint16_t*)(b + 6656 + 2 * li);
      }
    }
#pragma unroll
    for (int i = 0; i < NDMA; ++i) {
      if (4 * i + wv < (CPS * NPC + 63) / 64 && gst[i] < n)
        __builtin_amdgcn_global_load_lds((const void*)(XQ + goff[i] + 292L * (base + gst[i])),
                                         (__attribute__((address_space(3))) void*)(act + 1024 * (4 * i + wv)), 16,
                                         0, 0);
    }
    __builtin_amdgcn_s_waitcnt(0);  // every weight register and DMA piece of the group
    __syncthreads();
#pragma unroll
    for (int s = 0; s < CPS; ++s)
      if (s < n) {
        const uint8_t* As = act + s * STAGE;
        QHIP_Q6K_SUPERBLOCK(wr[s], As, arow);
      }
    __syncthreads();  // the next group's DMA overwrites the stages
  }
  mmq_write_tile<1, 1, 4, NE>(acc, Y, rows, tokens, r0, 0, 32 * wv, 0, tile, ksplit, ks, part, cnt);
}

// One thread per (tile, lane L) of the Q6_K fragment image: lane L's 96 quant
// bytes; lanes L < 32 also the row's scales and d.  Rows past the end: zeros.
__device__ __forceinline__ uint32_t ld32_bytes(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
__global__ __launch_bounds__(256) void k_wd_prepare_q6k(const uint8_t* __restrict__ W, uint8_t* __restrict__ IMG,
                                                         int rows, long row_bytes, int nsb, long nthreads) {
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= nthreads) return;
  const int L = (int)(gid & 63), i = L & 31, k = L >> 5;
  const long tile = gid >> 6;  // group * nsb + sb
  const long grp = tile / nsb;
  const int sb = (int)(tile - grp * nsb);
  const long row = grp * 32 + i;
  uint8_t* t = IMG + tile * kWdiTile;
  uint32_t q[24];
  uint32_t sc[4] = {0, 0, 0, 0}, d = 0;
  if (row < rows) {
    const uint8_t* b = W + row * row_bytes + 210L * sb;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int h = j >> 1, m = j & 1;
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        q[6 * j + w] = ld32_bytes(b + 64 * h + 16 * m + 8 * k + 4 * w);
        q[6 * j + 2 + w] = ld32_bytes(b + 64 * h + 32 + 16 * m + 8 * k + 4 * w);
        q[6 * j + 4 + w] = ld32_bytes(b + 128 + 32 * h + 16 * m + 8 * k + 4 * w);
      }
    }
#pragma unroll
    for (int w = 0; w < 4; ++w) sc[w] = ld32_bytes(b + 192 + 4 * w);
    d = (uint32_t)b[208] | ((uint32_t)b[209] << 8);
  } else {
#pragma unroll
    for (int w = 0; w < 24; ++w) q[w] = 0;
  }
#pragma unroll
  for (int c = 0; c < 6; ++c) *(uint4*)(t + 1024 * c + 16 * L) = make_uint4(q[4 * c], q[4 * c + 1], q[4 * c + 2], q[4 * c + 3]);
  if (k == 0) {
    *(uint4*)(t + 6144 + 16 * i) = make_uint4(sc[0], sc[1], sc[2], sc[3]);
    *(uint16_t*)(t + 6656 + 2 * i) = (uint16_t)d;
  }
}

// One thread per (tile, lane L) of the Q4_K fragment image: lane L's four
// 16-byte qs pieces; lanes L < 32 also the row's header.  Rows past the end:
// zeros.  GGUF Q4_K rows are 144 bytes per super-block: every piece aligned.
__global__ __launch_bounds__(256) void k_wd_prepare_q4k(const uint8_t* __restrict__ W, uint8_t* __restrict__ IMG,
                                                         int rows, long row_bytes, int nsb, long nthreads) {
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= nthreads) return;
  const int L = (int)(gid & 63), i = L & 31, k = L >> 5;
  const long tile = gid >> 6;  // group * nsb + sb
  const long grp = tile / nsb;
  const int sb = (int)(tile - grp * nsb);
  const long row = grp * 32 + i;
  uint8_t* t = IMG + tile * kWdiTile4;
  uint4 q[4], h = make_uint4(0u, 0u, 0u, 0u);
  if (row < rows) {
    const uint8_t* b = W + row * row_bytes + 144L * sb;
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = *(const uint4*)(b + 16 + 32 * c + 16 * k);
    h = *(const uint4*)b;
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) q[c] = make_uint4(0u, 0u, 0u, 0u);
  }
#pragma unroll
  for (int c = 0; c < 4; ++c) *(uint4*)(t + 1024 * c + 16 * L) = q[c];
  if (k == 0) *(uint4*)(t + 4096 + 16 * i) = h;
}

// ---- Q8_0 fragment image and its MMQ ----------------------------------------------------
// Image of a Q8_0 weight: per 32-row group, with nb = cols / 32 blocks, nb
// 1024-byte quant tiles (block b's tile: lane L's 16 bytes at 16 L are row
// L % 32, values 16 (L / 32)..+15, the MFMA operand fragment), then nb runs of
// the 32 rows' f16 scales in accumulator order (position 16 h + 4 q + i holds
// row 8 q + 4 h + i: the rows a lane with h = lane / 32 holds in its result
// elements 4 q + i).  1088 bytes per group and block, the GGUF rows' size.
constexpr int kQ8iBlk = 1088;
constexpr int kQ8iRow = 1040;  // LDS bytes per staged token row: 32 blocks + 16 (rows 4 banks apart)

__device__ __forceinline__ int q8i_pos(int i) { return 16 * ((i >> 2) & 1) + 4 * (i >> 3) + (i & 3); }
// staging unit u (TK tokens x 16 block pairs) -> token, pair
template <int TK>
__device__ __forceinline__ int q8i_unit_tok(int u) { return (u & 3) + 4 * ((u >> 4) & (TK / 4 - 1)); }
template <int TK>
__device__ __forceinline__ int q8i_unit_pair(int u) { return ((u >> 2) & 3) + 4 * (u / (4 * TK)); }

// One thread per (group, block, lane L): lane L's 16 quant bytes (2-byte
// aligned in the 34-byte GGUF block, read bytewise); lanes L < 32 also the
// row's scale.  Rows past the end: zeros.
__global__ __launch_bounds__(256) void k_wd_prepare_q8(const uint8_t* __restrict__ W, uint8_t* __restrict__ IMG,
                                                        int rows, long row_bytes, int nb, long nthreads) {
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= nthreads) return;
  const int L = (int)(gid & 63), i = L & 31, k = L >> 5;
  const long tile = gid >> 6;  // group * nb + b
  const long grp = tile / nb;
  const int b = (int)(tile - grp * nb);
  const long row = grp * 32 + i;
  uint8_t* t = IMG + grp * nb * kQ8iBlk;
  uint32_t q[4] = {0, 0, 0, 0};
  uint16_t d = 0;
  if (row < rows) {
    const uint8_t* blk = W + row * row_bytes + 34L * b;
#pragma unroll
    for (int w = 0; w < 4; ++w) q[w] = ld32_bytes(blk + 2 + 16 * k + 4 * w);
    d = (uint16_t)(blk[0] | (blk[1] << 8));
  }
  *(uint4*)(t + 1024L * b + 16 * L) = make_uint4(q[0], q[1], q[2], q[3]);
  if (k == 0) *(uint16_t*)(t + 1024L * nb + 64L * b + 2 * q8i_pos(i)) = d;
}

// Q8_0 MMQ from the fragment image (cols a multiple of 256).  A workgroup of
// eight waves owns 64 rows x 32 NG tokens; wave w takes row group w & 1 and
// K quarter w >> 1 of each 32-block super-chunk.  Operand A is the weights,
// loaded from the image straight into registers; operand B the activations,
// copied from the Q8_0 rows into LDS once per workgroup (1040-byte token
// rows, the block scales apart as f16).  So every lane holds one token and 16
// rows: its activation scale is one value per block, the 16 weight scales are
// read from an f32 LDS plane in accumulator order.  Per block the MFMA result
// read as a float is 1.5 2^23 + sumi (exact, |sumi| <= 2^19) and
//   t = fma(F, da, -1.5 2^23 da) = da sumi,   acc = fma(t, dw, acc)
// (kernels32.c:447-464: sumi * (dw * da), here rounded as (da * sumi) * dw).
// At the end the four K quarters' partial tiles are added through LDS in
// quarter order, so the result does not depend on timing.
// Occupancy: two workgroups per CU (under 80 KB of LDS each, at most 128
// VGPRs), four waves per SIMD.
template <int NG, bool ONE, bool FULL>
__global__ __launch_bounds__(512, 4) void k_mmq_q8i(const uint8_t* __restrict__ IMG, const uint8_t* __restrict__ XQ,
                                                     float* __restrict__ Y, int rows, int tokens, int nb,
                                                     long act_bytes, int ntt) {
  constexpr int TK = 32 * NG;  // tokens per tile
  constexpr int AQ = TK * kQ8iRow, DAH = 4 * TK * 16, DWF = 32 * 2 * 32 * 4;
  constexpr int PRT = 2 * 4 * TK * 36 * 4;  // partial tiles [row group][quarter][token][36]
  constexpr int LDSB = AQ + DAH + DWF > PRT ? AQ + DAH + DWF : PRT;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDSB];
  uint8_t* aq = lds;
  uint8_t* dah = lds + AQ;  // [block / 8][token][8] f16
  float* dwf = (float*)(lds + AQ + DAH);  // [block][row group][32] in accumulator order

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 31, lh = lane >> 5;
  const int rg = wv & 1, kq = wv >> 1;
  const int G = gridDim.x;
  int g = blockIdx.x;
  if ((G & 7) == 0) g = (g & 7) * (G >> 3) + (g >> 3);
  const int rt = g / ntt, t0 = (g - rt * ntt) * TK;
  const int ngrp = (rows + 31) >> 5;
  const long gbytes = (long)nb * kQ8iBlk;
  const int grp = 2 * rt + rg;
  const uint8_t* wimg = IMG + (long)(grp < ngrp ? grp : ngrp - 1) * gbytes;

  f32x16 acc[NG];
#pragma unroll
  for (int a = 0; a < NG; ++a)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[a][e] = 0.0f;
  i32x16 bias;
#pragma unroll
  for (int e = 0; e < 16; ++e) bias[e] = kBiasBits;
  asm volatile("" : "+v"(bias));

  // ONE: the launch guarantees nb <= 32 (one super-chunk, so nothing but the
  // bias is live across the staging: 64 tokens fit the register budget)
  const int nbl = ONE ? 32 : nb;
  for (int sc0 = 0; sc0 < nbl && sc0 < nb; sc0 += 32) {
    const int n = nb - sc0 < 32 ? nb - sc0 : 32;  // a multiple of 8
    const int q4 = FULL ? 8 : n >> 2, bl0 = kq * q4;  // FULL: nb % 32 == 0
    // this wave's first two weight fragments, then the activation and scale
    // loads of the whole workgroup
    u32x4 wf[3];
    const uint8_t* wq = wimg + 1024L * (sc0 + bl0) + 16 * lane;
    wf[0] = *(const u32x4*)wq;
    wf[1] = *(const u32x4*)(wq + 1024);
    // activation unit u = tid + 512 i: blocks 2 p, 2 p + 1 of one token, 68
    // bytes from a 4-byte aligned address.  Sixteen consecutive lanes take 4
    // tokens x 4 pairs (unit_tok / unit_pair): their 16-byte LDS writes land
    // in 16 different bank groups (token rows are 65 groups apart), and each
    // token's 4 pairs are 272 contiguous bytes of the row.
    uint32_t x[NG][17];
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int u = tid + 512 * i, tok = q8i_unit_tok<TK>(u), p = q8i_unit_pair<TK>(u);
      const int tt = t0 + tok < tokens ? t0 + tok : tokens - 1;
      const uint8_t* src = XQ + (long)tt * act_bytes + 34L * (sc0 + 2 * (2 * p < n ? p : 0));
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32x4 v = *(const u32x4*)(src + 16 * c);
        x[i][4 * c] = v.x; x[i][4 * c + 1] = v.y; x[i][4 * c + 2] = v.z; x[i][4 * c + 3] = v.w;
      }
      x[i][16] = *(const uint32_t*)(src + 64);
    }
    // weight scales: thread tid < 256 converts 8 of one row group's block
    u32x4 ws = {0u, 0u, 0u, 0u};
    const int spart = tid & 3, sr = (tid >> 2) & 1, sbl = tid >> 3;
    const int sgrp = 2 * rt + sr;
    if (tid < 256 && sbl < n)
      ws = *(const u32x4*)(IMG + (long)(sgrp < ngrp ? sgrp : ngrp - 1) * gbytes + 1024L * nb + 64L * (sc0 + sbl) +
                           16 * spart);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int u = tid + 512 * i, tok = q8i_unit_tok<TK>(u), p = q8i_unit_pair<TK>(u);
      if (2 * p < n) {
        uint32_t q0[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) q0[j] = __builtin_amdgcn_alignbyte(x[i][j + 1], x[i][j], 2);
        uint8_t* dst = aq + tok * kQ8iRow + 64 * p;
        st16(dst, q0[0], q0[1], q0[2], q0[3]);
        st16(dst + 16, q0[4], q0[5], q0[6], q0[7]);
        st16(dst + 32, x[i][9], x[i][10], x[i][11], x[i][12]);
        st16(dst + 48, x[i][13], x[i][14], x[i][15], x[i][16]);
        *(uint32_t*)(dah + ((p >> 2) * TK + tok) * 16 + 4 * (p & 3)) = (x[i][0] & 0xFFFFu) | (x[i][8] & 0xFFFF0000u);
      }
    }
    if (tid < 256 && sbl < n) {
      const uint32_t h[4] = {ws.x, ws.y, ws.z, ws.w};
      float f[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[2 * j] = h2f(h[j] & 0xFFFFu);
        f[2 * j + 1] = h2f(h[j] >> 16);
      }
      float* dst = dwf + (sbl * 2 + sr) * 32 + 8 * spart;
      *(f32x4*)dst = f32x4{f[0], f[1], f[2], f[3]};
      *(f32x4*)(dst + 4) = f32x4{f[4], f[5], f[6], f[7]};
    }
    __syncthreads();

#pragma unroll
    for (int s = 0; s < 8; ++s) {
      if (s < q4) {
        if (s + 2 < q4) wf[(s + 2) % 3] = *(const u32x4*)(wq + 1024L * (s + 2));
        const int bl = bl0 + s;
        i32x16 c[NG];
#pragma unroll
        for (int a = 0; a < NG; ++a) {
          const i32x4 af = *(const i32x4*)(aq + (32 * a + li) * kQ8iRow + 32 * bl + 16 * lh);
          const u32x4 w = wf[s % 3];
          c[a] = __builtin_amdgcn_mfma_i32_32x32x32_i8(i32x4{(int)w.x, (int)w.y, (int)w.z, (int)w.w}, af, bias, 0,
                                                        0, 0);
        }
        float da[NG], nbd[NG];
#pragma unroll
        for (int a = 0; a < NG; ++a) {
          da[a] = h2f(*(const uint16_t*)(dah + ((bl >> 3) * TK + 32 * a + li) * 16 + 2 * (bl & 7)));
          nbd[a] = -kBias * da[a];
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const f32x4 dw = *(const f32x4*)(dwf + (bl * 2 + rg) * 32 + 16 * lh + 4 * q);
#pragma unroll
          for (int a = 0; a < NG; ++a)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int ce = c[a][4 * q + i];
              const float t = __builtin_fmaf(__int_as_float(ce), da[a], nbd[a]);
              acc[a][4 * q + i] = __builtin_fmaf(t, dw[i], acc[a][4 * q + i]);
            }
        }
      }
    }
    __syncthreads();  // the next super-chunk (or the partial tiles) overwrites the stages
  }

  // partial tiles, then the sum over the quarters in quarter order
  float* prt = (float*)lds;
#pragma unroll
  for (int a = 0; a < NG; ++a)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *(f32x4*)(prt + ((rg * 4 + kq) * TK + 32 * a + li) * 36 + 8 * q + 4 * lh) =
          f32x4{acc[a][4 * q], acc[a][4 * q + 1], acc[a][4 * q + 2], acc[a][4 * q + 3]};
  __syncthreads();
  const int orr = wv >> 2, tb = wv & 3, rq = lane & 7, tl = lane >> 3;
#pragma unroll
  for (int m = 0; m < NG; ++m) {
    const int tok = 8 * NG * tb + 8 * m + tl;
    const float* pp = prt + (orr * 4 * TK + tok) * 36 + 4 * rq;
    f32x4 v = *(const f32x4*)pp;
#pragma unroll
    for (int k = 1; k < 4; ++k) v += *(const f32x4*)(pp + k * TK * 36);
    const int row = 32 * (2 * rt + orr) + 4 * rq;
    if (t0 + tok < tokens) {
      float* yo = Y + (long)(t0 + tok) * rows + row;
      if (row < rows) yo[0] = v.x;
      if (row + 1 < rows) yo[1] = v.y;
      if (row + 2 < rows) yo[2] = v.z;
      if (row + 3 < rows) yo[3] = v.w;
    }
  }
}

static hipError_t launch_mmq_q8i(const GemvArgs& g, hipStream_t s) {
  const int nb = g.cols / 32;
  const long ntr = (g.rows + 63) / 64;
  // 64-token tiles where K is one super-chunk (up to 1024 values) and they
  // still give at least 1.75 workgroups per CU, else 32.  Measured on
  // MI355X, [3584, 1024]: 64 / 96 / 128 / 256 tokens 5.0 / 5.1 / 5.2 / 7.1 us
  // with 32-token tiles against 7.0 / 7.1 / 7.1 / 7.7 with 64; 512 tokens
  // (448 tiles of 64) 11.5 against 12.3; [6144, 1024] x 200 9.9 against 11.1
  const int cus = qhip_gpu_cu_count() > 0 ? qhip_gpu_cu_count() : 256;
  const int tk = g.tokens > 32 && nb <= 32 && ntr * ((g.tokens + 63) / 64) * 4 >= 7L * cus ? 64 : 32;
  const long ntt = (g.tokens + tk - 1) / tk;
  const long G = ntr * ntt;
  if (G > 0x7FFFFFFFL || g.act_bytes != 34L * nb) return hipErrorInvalidValue;
#define QHIP_Q8I(NG, ONE, FULL)                                                                               \
  hipLaunchKernelGGL((k_mmq_q8i<NG, ONE, FULL>), dim3((unsigned)G), dim3(512), 0, s, (const uint8_t*)g.w,       \
                     (const uint8_t*)g.xq, g.out, g.rows, g.tokens, nb, g.act_bytes, (int)ntt)
  const bool full = nb % 32 == 0;
  if (tk == 32) {
    if (full) QHIP_Q8I(1, false, true);
    else QHIP_Q8I(1, false, false);
  } else {
    if (full) QHIP_Q8I(2, true, true);
    else QHIP_Q8I(2, true, false);
  }
#undef QHIP_Q8I
  return hipGetLastError();
}

// ---- Q6_K MMQ from the plane image (long prompts) ---------------------------------------
// The plane image of a Q6_K weight holds p = sc (q6 - 32) for every value
// (kernels256.c:200-212, :720-738: q6 from ql and qh, sc the 16-value
// group's int8 scale) split exactly as p = 64 hi + lo (lo = p & 63, hi = p >> 6
// >= -64), both planes in MFMA fragment order: per 32-row group and
// super-block, 8 KB of hi fragments (sub-block s at 1024 s, lane L's 16 bytes
// at 16 L: row L % 32, values 32 s + 16 (L / 32) ..+15), 8 KB of lo fragments,
// then the 32 rows' f32 scales d -- 16,512 bytes per 32 rows and 256 values,
// 2.5x the GGUF bytes.  Every weight load is one aligned, contiguous 1 KB.
//
// Tiles of 128 rows x TK = 32 NA tokens.  Within a workgroup of four waves,
// wave w takes row group w and all TK tokens as NA 32 x 32 tiles, so each
// plane fragment feeds NA MFMAs.  Each tile has ONE integer accumulator: the
// eight hi-plane MFMAs of a super-block run first, the accumulator is shifted
// left by six, then the eight lo-plane MFMAs chain onto it, so it ends as
// isum = 64 C_hi + C_lo, the reference's per-super-block integer exactly
// (|isum| < 2^27).  Each plane fragment's register is reloaded with the next
// unit's fragment as soon as its MFMAs are issued, so the weights need no
// second register set.  Activations: the tile's TK Q8_K rows of one
// super-block are copied into LDS by global_load_lds (double buffered): the
// quants as 256-byte token rows with the 16-byte slots XOR-swizzled by the
// token index (every copy instruction reads 4 tokens' contiguous 256 bytes;
// every MFMA operand read is conflict free), the f32 scales packed.
//
// Work distribution (the grid is persistent: two workgroups per CU).  The
// unit of work is one tile x one super-block.  With N workgroups and ntiles
// tiles, the first N floor(ntiles / N) tiles are whole tiles, workgroup L
// taking tiles L, L + N, ... (so at any time the workgroups on one XCD work
// on neighbouring tiles: the token tiles of one row tile, which share the
// weights); the remaining tiles are cut into P slices over K, which the
// workgroups take after their whole tiles, piece L + N r to workgroup L.  P
// minimises the work of the busiest workgroup (at least four super-blocks a
// slice), and the pieces are ordered (group of ntt tiles, slice, tile) so
// that the pieces running side by side read the same weights -- with the
// pieces of one tile at different K they would each stream the weights.  A
// sliced tile is finished deterministically: each slice writes its partial
// tile to the workspace, the last to arrive adds the P partials in slice
// order and writes the outputs.
constexpr int kBgQ6Grp = 16512;  // plane image bytes per 32-row group and super-block

struct BgPlan {
  int ntt, nsb, ntiles, nwg;
  int dpw;       // whole tiles per workgroup
  int sk_tiles;  // sliced tiles
  int P;         // slices per sliced tile
  int gw;        // sliced tiles per piece group
};

// piece p of the sliced tiles -> (sliced tile u, slice)
__device__ __forceinline__ void bg_piece(const BgPlan& q, int p, int& u, int& slice) {
  const int full = q.sk_tiles / q.gw, rem = q.sk_tiles - full * q.gw;
  if (p < full * q.P * q.gw) {
    const int g = p / (q.P * q.gw), loc = p - g * q.P * q.gw;
    slice = loc / q.gw;
    u = g * q.gw + loc % q.gw;
  } else {
    const int loc = p - full * q.P * q.gw;
    slice = loc / rem;
    u = full * q.gw + loc % rem;
  }
}
// the inverse
__device__ __forceinline__ int bg_piece_index(const BgPlan& q, int u, int slice) {
  const int full = q.sk_tiles / q.gw, rem = q.sk_tiles - full * q.gw;
  if (u < full * q.gw) return (u / q.gw) * q.P * q.gw + slice * q.gw + u % q.gw;
  return full * q.P * q.gw + slice * rem + (u - full * q.gw);
}

// The workgroup barrier between units: s_waitcnt vmcnt(N) lgkmcnt(0), then
// s_barrier.  Vector memory loads complete in issue order, so vmcnt(N) means
// everything but this wave's N most recent loads has landed; __syncthreads
// would wait for all of them (its release fence is vmcnt(0)).  The compiler
// barriers keep LDS accesses on their side of the s_barrier.
template <int N>
__device__ __forceinline__ void bg_sync() {
  static_assert(N >= 0 && N < 64, "vmcnt is six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Vector loads a wave of k_mmq_bg_q6k issues after a unit's activation copy:
// the 8 hi-plane and 8 lo-plane fragments of the next unit and its row scale.
constexpr int kBgLoadsAfterCopy = 2 * 8 + 1;

template <int NA>
__global__ __launch_bounds__(256, 2) void k_mmq_bg_q6k(const uint8_t* __restrict__ IMG, const uint8_t* __restrict__ XQ,
                                                        float* __restrict__ Y, int rows, int tokens, long act_bytes,
                                                        BgPlan P, float* __restrict__ part, unsigned* __restrict__ cnt) {
  constexpr int TK = 32 * NA, DYO = 256 * TK, STAGE = 260 * TK;
  constexpr long PT = 128L * TK;  // floats per partial tile
  __shared__ __attribute__((aligned(16))) uint8_t act[2][STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 31, lh = lane >> 5;
  int L = blockIdx.x;
  if ((P.nwg & 7) == 0) L = (L & 7) * (P.nwg >> 3) + (L >> 3);  // XCD-contiguous workgroups
  const int nsb = P.nsb, ngrp = (rows + 31) >> 5;
  const int dp_tiles = P.dpw * P.nwg, npieces = P.sk_tiles * P.P;
  // this workgroup's ranges: whole tiles L + N r (r < dpw), then pieces
  // L + N (r - dpw)
  const int nr = P.dpw + (L < npieces ? (npieces - L + P.nwg - 1) / P.nwg : 0);
  // a unit: range r, tile, its row tile, its token tile, super-block, the
  // range's end, its piece (-1 for a whole tile)
  struct U {
    int r, tile, rt, tt, sb, end, piece;
  };
  auto begin = [&](int r) -> U {
    U u;
    u.r = r;
    if (r < P.dpw) {
      u.tile = L + r * P.nwg;
      u.sb = 0;
      u.end = nsb;
      u.piece = -1;
    } else {
      int t, sl;
      u.piece = L + (r - P.dpw) * P.nwg;
      bg_piece(P, u.piece, t, sl);
      u.tile = dp_tiles + t;
      u.sb = sl * nsb / P.P;
      u.end = (sl + 1) * nsb / P.P;
    }
    u.rt = u.tile / P.ntt;
    u.tt = u.tile - u.rt * P.ntt;
    return u;
  };
  auto advance = [&](U u) -> U {
    if (u.sb + 1 < u.end) {
      ++u.sb;
      return u;
    }
    return begin(u.r + 1);
  };
  // The copy of a unit's activations.  Quants: instruction i of wave w copies
  // tokens 16 i + 4 w + 0..3, 16 lanes (256 contiguous bytes) each, into
  // 256-byte LDS rows, lane q of a token taking slot q ^ (token & 15) so that
  // 16 consecutive tokens' slot s lie in 16 different bank groups.  Scales:
  // one f32 per lane, the first NA / 2 waves.  Tokens past the end re-read
  // the last one.
  const int qtok = 4 * wv + (lane >> 4);
  const int qoff = 4 + 16 * ((lane & 15) ^ (qtok & 15));
  auto issue_act = [&](const U& u, uint8_t* st) {
    const int t0 = u.tt * TK, tl = tokens - 1 - t0;
    const uint8_t* base = XQ + (long)t0 * act_bytes + 292L * u.sb;
#pragma unroll
    for (int i = 0; i < TK / 16; ++i) {
      const int tk = 16 * i + qtok < tl ? 16 * i + qtok : tl;
      const uint8_t* src = base + (long)tk * act_bytes + qoff;
      uint8_t* dst = st + 1024 * (4 * i + wv);
      if constexpr (NA == 4) lds_copy16(src, dst);
      else __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
    }
    if (wv < NA / 2) {
      const int tk = 64 * wv + lane < tl ? 64 * wv + lane : tl;
      const uint8_t* src = base + (long)tk * act_bytes;
      uint8_t* dst = st + DYO + 256 * wv;
      if constexpr (NA == 4) lds_copy4(src, dst);
      else __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)dst, 4, 0, 0);
    }
  };
  // this wave's 32-row group of unit u in the image (a group past the end
  // re-reads the last)
  auto wgrp = [&](const U& u) -> const uint8_t* {
    const int grp = 4 * u.rt + wv < ngrp ? 4 * u.rt + wv : ngrp - 1;
    return IMG + ((long)grp * nsb + u.sb) * kBgQ6Grp;
  };
  auto afrag = [&](const uint8_t* A, int a, int s) -> i32x4 {
    return *(const i32x4*)(A + 256 * (32 * a + li) + 16 * ((2 * s + lh) ^ (li & 15)));
  };

  f32x16 acc[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[a][e] = 0.0f;
  i32x16 zero = {};
  asm volatile("" : "+v"(zero));  // one register block used as every first C operand
  // the current unit's 16 plane fragments and row scale
  i32x4 ph[8], pq[8];
  float dw;
  if (nr == 0) return;  // uniform over the workgroup
  U cu = begin(0);
  issue_act(cu, &act[0][0]);
  {
    const uint8_t* b = wgrp(cu);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      ph[s] = *(const i32x4*)(b + 1024 * s + 16 * lane);
      pq[s] = *(const i32x4*)(b + 8192 + 1024 * s + 16 * lane);
    }
    dw = *(const float*)(b + 16384 + 4 * li);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int k = 0;; ++k) {
    const bool more = cu.sb + 1 < cu.end || cu.r + 1 < nr;
    const U nu = more ? advance(cu) : cu;  // the last unit re-reads its own operands
    const uint8_t* A = &act[k & 1][0];
    issue_act(nu, &act[(k & 1) ^ 1][0]);
    // no load of the next unit's weights may be issued ahead of the copy:
    // the barrier below counts them as the last kBgLoadsAfterCopy loads
    asm volatile("" ::: "memory");
    const uint8_t* nb = wgrp(nu);
    i32x16 is[NA];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int a = 0; a < NA; ++a)
        is[a] = __builtin_amdgcn_mfma_i32_32x32x32_i8(afrag(A, a, s), ph[s], s == 0 ? zero : is[a], 0, 0, 0);
      ph[s] = *(const i32x4*)(nb + 1024 * s + 16 * lane);
    }
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int e = 0; e < 16; ++e) is[a][e] <<= 6;
    // the lo pass reads the same LDS operands again: without this the
    // compiler keeps the hi pass's fragments live instead
    asm volatile("" ::: "memory");
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
      for (int a = 0; a < NA; ++a) is[a] = __builtin_amdgcn_mfma_i32_32x32x32_i8(afrag(A, a, s), pq[s], is[a], 0, 0, 0);
      pq[s] = *(const i32x4*)(nb + 8192 + 1024 * s + 16 * lane);
    }
    const float d = dw;
    dw = *(const float*)(nb + 16384 + 4 * li);
    // acc += dy * (d * isum): lane element e holds token 8 (e / 4) + 4 (lane /
    // 32) + e % 4 of its tile
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 dy = *(const f32x4*)(A + DYO + 4 * (32 * a + 8 * q + 4 * lh));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int e = 4 * q + i;
          acc[a][e] = __builtin_fmaf(dy[i], d * (float)is[a][e], acc[a][e]);
        }
      }
    if (!more || nu.r != cu.r) {
      // the range ends here: a whole tile, or one slice of a sliced tile
      const int row = 128 * cu.rt + 32 * wv + li, t0 = cu.tt * TK;
      bool direct = cu.piece < 0 || P.P == 1;
      if (!direct) {
        float* pp = part + (long)cu.piece * PT + (long)wv * (1024 * NA) + lane;
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int e = 0; e < 16; ++e) sk_store(pp + (a * 16 + e) * 64, acc[a][e]);
        const int u = cu.tile - dp_tiles;
        unsigned* tc = cnt + u;
        if (sk_arrive(tc, (unsigned)P.P)) {
#pragma unroll
          for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[a][e] = 0.0f;
          for (int sl = 0; sl < P.P; ++sl) {
            const float* qq = part + (long)bg_piece_index(P, u, sl) * PT + (long)wv * (1024 * NA) + lane;
#pragma unroll
            for (int a = 0; a < NA; ++a) {
              float v[16];
#pragma unroll
              for (int e = 0; e < 16; ++e) v[e] = sk_load(qq + (a * 16 + e) * 64);
#pragma unroll
              for (int e = 0; e < 16; ++e) acc[a][e] += v[e];
            }
          }
          sk_reset(tc);
          direct = true;
        }
      }
      if (direct) {
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int t = t0 + 32 * a + 8 * (e >> 2) + 4 * lh + (e & 3);
            if (row < rows && t < tokens) Y[(long)t * rows + row] = acc[a][e];
          }
      }
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[a][e] = 0.0f;
    }
    // unit k+1's activations are in LDS once this wave's copy has landed;
    // the weight loads issued after it (8 hi-plane and 8 lo-plane fragments,
    // the row scale) may stay in flight
    bg_sync<kBgLoadsAfterCopy>();
    if (!more) break;
    cu = nu;
  }
}

// One thread per (32-row group, super-block, sub-block s, lane L): the 16
// values 32 s + 16 (L / 32) .. +15 of row 32 group + L % 32 as both planes,
// and for s = 0 the row's f32 scale.  Rows past the end: zeros.
__global__ __launch_bounds__(256) void k_bg_prepare_q6k(const uint8_t* __restrict__ W, uint8_t* __restrict__ IMG,
                                                         int rows, long row_bytes, int nsb, long nthreads) {
  const long gid = (long)blockIdx.x * 256 + threadIdx.x;
  if (gid >= nthreads) return;
  const int Lq = (int)(gid & 63), s = (int)((gid >> 6) & 7);
  const long gs = gid >> 9;  // group * nsb + sb
  const long grp = gs / nsb;
  const int sb = (int)(gs - grp * nsb);
  const long row = grp * 32 + (Lq & 31);
  const int e0 = 32 * s + 16 * (Lq >> 5);
  uint32_t hi[4] = {0, 0, 0, 0}, lo[4] = {0, 0, 0, 0};
  float d = 0.0f;
  if (row < rows) {
    const uint8_t* blk = W + row * row_bytes + 210L * sb;
    const int sc = (int)(int8_t)blk[192 + (e0 >> 4)];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int e = e0 + i, h = e >> 7, q = (e & 127) >> 5, l = e & 31;
      uint32_t lq = blk[64 * h + 32 * (q & 1) + l];
      lq = q >= 2 ? (lq >> 4) : (lq & 15u);
      const uint32_t hb = (blk[128 + 32 * h + l] >> (2 * q)) & 3u;
      const int pv = sc * ((int)(lq | (hb << 4)) - 32);
      hi[i >> 2] |= ((uint32_t)(pv >> 6) & 255u) << (8 * (i & 3));  // arithmetic shift: floor
      lo[i >> 2] |= (uint32_t)(pv & 63) << (8 * (i & 3));
    }
    d = h2f((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
  }
  uint8_t* b = IMG + gs * kBgQ6Grp;
  *(uint4*)(b + 1024 * s + 16 * Lq) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  *(uint4*)(b + 8192 + 1024 * s + 16 * Lq) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  if (s == 0 && Lq < 32) *(float*)(b + 16384 + 4 * Lq) = d;
}

long bg_image_bytes_q6k(int rows, int cols) {
  if (rows < 0 || cols <= 0 || cols % 256) return -1;
  return (long)((rows + 31) / 32) * (cols / 256) * kBgQ6Grp;
}

hipError_t launch_bg_prepare_q6k(const void* w, long row_bytes, int rows, int cols, void* img, hipStream_t s) {
  if (bg_image_bytes_q6k(rows, cols) < 0) return hipErrorInvalidValue;
  const long n = (long)((rows + 31) / 32) * (cols / 256) * 512;
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_bg_prepare_q6k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint8_t*)w,
                     (uint8_t*)img, rows, row_bytes, cols / 256, n);
  return hipGetLastError();
}

// Token tiles of the plane-image MMQ: 64 tokens up to 192, else 128.
// Measured on MI355X, [5120, 17408]: 64.3 / 64.7 / 78.1 / 101.1 / 108.6 /
// 144.5 us at 160 / 192 / 256 / 320 / 384 / 512 tokens with 64-token tiles,
// 74.8 / 72.9 / 75.7 / 96.1 / 95.7 / 123.3 with 128-token tiles.
static int bg_na(const GemvArgs& g) { return g.tokens <= 192 ? 2 : 4; }

// split = false: no tile is cut over K (no workspace needed)
static BgPlan bg_plan(const GemvArgs& g, int nwg, bool split) {
  BgPlan p{};
  const int tk = 32 * bg_na(g);
  p.nsb = g.cols / 256;
  p.ntt = (g.tokens + tk - 1) / tk;
  p.ntiles = p.ntt * ((g.rows + 127) / 128);
  if (nwg <= 0) {
    const int cus = qhip_gpu_cu_count();
    nwg = 2 * (cus > 0 ? cus : 256);  // two workgroups per CU
  }
  p.nwg = nwg;
  p.dpw = p.ntiles / p.nwg;
  p.sk_tiles = p.ntiles - p.dpw * p.nwg;
  p.P = 1;
  p.gw = 1;
  if (p.sk_tiles > 0 && split && p.sk_tiles <= kSkMaxTiles) {
    // the slice count with the least work on the busiest workgroup (ties:
    // fewer slices), at least four super-blocks a slice; a slice costs its
    // super-blocks plus about two for writing and adding its partial tile
    long best = -1;
    const int pmax = p.nsb / 4 > 1 ? p.nsb / 4 : 1;
    for (int q = 1; q <= pmax && q <= 64; ++q) {
      const long per = (long)p.sk_tiles * q;
      const long m = ((per + p.nwg - 1) / p.nwg) * ((p.nsb + q - 1) / q + (q > 1 ? 2 : 0));
      if (best < 0 || m < best) {
        best = m;
        p.P = q;
      }
    }
    p.gw = p.ntt < p.sk_tiles ? p.ntt : p.sk_tiles;
  }
  if (p.dpw == 0 && (long)p.sk_tiles * p.P < p.nwg) p.nwg = p.sk_tiles * p.P;  // no workgroup without work
  return p;
}

// Workspace of the plane-image MMQ: tile counters, then one partial tile per
// piece (none when no tile is sliced).
long bg_work_bytes(const GemvArgs& g, int nwg) {
  if (g.rows <= 0 || g.tokens <= 0 || g.cols <= 0 || g.cols % 256) return 0;
  const BgPlan p = bg_plan(g, nwg, true);
  if (p.P <= 1) return 0;
  return kSkCountBytes + (long)p.sk_tiles * p.P * 128L * 32 * bg_na(g) * 4;
}

// g.w: the Q6_K plane image; nwg > 0 overrides the persistent grid.  Without
// a workspace of bg_work_bytes no tile is cut over K.
hipError_t launch_mmq_bg_q6k(const GemvArgs& g, void* work, long work_bytes, hipStream_t s, int nwg) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  if (g.ttype != TT_Q6_K || g.cols % 256 || g.act_bytes != 292L * (g.cols / 256) ||
      (long)g.tokens * g.act_bytes > 0x7FFFFFFFL || (long)g.tokens * ((g.rows + 127) / 128) > 0x3FFFFFFFL)
    return hipErrorInvalidValue;
  const long need = bg_work_bytes(g, nwg);
  const BgPlan p = bg_plan(g, nwg, need > 0 && work && work_bytes >= need);
  unsigned* cnt = (unsigned*)work;
  float* part = work ? (float*)((uint8_t*)work + kSkCountBytes) : nullptr;
  if (bg_na(g) == 2)
    hipLaunchKernelGGL(k_mmq_bg_q6k<2>, dim3((unsigned)p.nwg), dim3(256), 0, s, (const uint8_t*)g.w,
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.act_bytes, p, part, cnt);
  else
    hipLaunchKernelGGL(k_mmq_bg_q6k<4>, dim3((unsigned)p.nwg), dim3(256), 0, s, (const uint8_t*)g.w,
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.act_bytes, p, part, cnt);
  return hipGetLastError();
}

long wd_image_bytes(int ttype, int rows, int cols) {
  if ((ttype != TT_Q6_K && ttype != TT_Q4_K && ttype != TT_Q8_0) || rows < 0 || cols <= 0 || cols % 256) return -1;
  if (ttype == TT_Q8_0) return (long)((rows + 31) / 32) * (cols / 32) * kQ8iBlk;
  return (long)((rows + 31) / 32) * (cols / 256) * (ttype == TT_Q6_K ? kWdiTile : kWdiTile4);
}

hipError_t launch_wd_prepare(int ttype, const void* w, long row_bytes, int rows, int cols, void* img,
                             hipStream_t s) {
  if (wd_image_bytes(ttype, rows, cols) < 0) return hipErrorInvalidValue;
  const int nsb = cols / 256;
  if (ttype == TT_Q8_0) {
    const long n8 = (long)((rows + 31) / 32) * (cols / 32) * 64;
    if (n8 == 0) return hipSuccess;
    hipLaunchKernelGGL(k_wd_prepare_q8, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, s, (const uint8_t*)w,
                       (uint8_t*)img, rows, row_bytes, cols / 32, n8);
    return hipGetLastError();
  }
  const long n = (long)((rows + 31) / 32) * nsb * 64;
  if (n == 0) return hipSuccess;
  if (ttype == TT_Q6_K)
    hipLaunchKernelGGL(k_wd_prepare_q6k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint8_t*)w,
                       (uint8_t*)img, rows, row_bytes, nsb, n);
  else
    hipLaunchKernelGGL(k_wd_prepare_q4k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, (const uint8_t*)w,
                       (uint8_t*)img, rows, row_bytes, nsb, n);
  return hipGetLastError();
}

// ---- few tokens, K split inside the workgroup -------------------------------------------
// T <= 8 NG from a fragment image with no split-K hand-off between
// workgroups: a workgroup of NW waves owns one group of 32 rows; wave w takes
// super-blocks [w cpw, (w+1) cpw) of the whole row (its own activation stages
// in LDS, its weight loads and DMA for CPS super-blocks issued before any of
// it is used), and the waves' partial sums are added through LDS in wave
// order by wave 0, which writes the outputs.  The hand-off of the split
// launches (partials written through to the coherence point, a counter
// round trip, the last workgroup reading every slice back) costs 3.5-4 us at
// config 5 whatever the token count; here the sum stays in the workgroup.
// Measured on MI355X (one weight copy, read from the Infinity Cache), config
// 5, 1 / 8 / 16 / 24 tokens: Q4_K [17408, 5120] with 4 waves 10.6 / 11.4 /
// 13.1 / 17.1 us (2 / 3 / 5 / 6 / 8 waves: 13.4 /
// 11.6 / 11.2 / 11.2 / 11.7 us at 1 token), against 14.5 / 14.7 / 15.8 / 20.0
// for the split launches; Q6_K [5120, 17408] (160 groups) with 12 waves
// 17.3 / 17.8 / 22.6 / 28.3 us (8 / 10 / 14 / 16 waves: 19.4 / 18.9 / 18.9 /
// 18.8 at 1 token), against 20.9 / 21.2 / 24.0 / 27.8.  One super-block per
// load round (CPS = 1) beats whole groups of 2-5 (Q4_K 11.6-15.4 us at 1
// token): fewer registers, more waves resident.  With the weights streamed
// from HBM (rotated copies) the same choices win: Q4_K 12.6 / 14.2 us at 1 / 8
// tokens (3 / 6 / 8 waves 13.8 / 13.3 / 13.8 at 1 token; two super-blocks per
// round 14.7), Q6_K 19.6 / 21.0 (8 / 16 waves 22.5 / 25.9).
template <int TT, int NG, int NW, int CPS>
__global__ __launch_bounds__(64 * NW) void k_mmq_rk(const uint8_t* __restrict__ W, const uint8_t* __restrict__ XQ,
                                                     float* __restrict__ Y, int rows, int tokens, long act_bytes,
                                                     int nsb, int cpw) {
  constexpr int TR = 8 * NG, NE = 4 * NG;
  constexpr int STAGE = TR * kWdRow, NPC = TR * kWdPieces, NDW = (CPS * NPC + 63) / 64;
  constexpr int TILE = TT == TT_Q6_K ? kWdiTile : kWdiTile4;
  constexpr int LDSB = NW * CPS * STAGE > NW * NE * 256 ? NW * CPS * STAGE : NW * NE * 256;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDSB];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, li = lane & 31, lh = lane >> 5;
  const int grp = blockIdx.x, ngrp = (rows + 31) >> 5;
  const uint8_t* wbase = W + (long)(grp < ngrp ? grp : ngrp - 1) * nsb * TILE;
  const int sb0 = wv * cpw, sb1 = sb0 + cpw < nsb ? sb0 + cpw : nsb;
  const int arow = li < TR ? li : 0;
  uint8_t* act = lds + wv * CPS * STAGE;  // this wave's stages

  // DMA piece P = 64 i + lane of this wave's run: stage P / (19 TR), token
  // row (P % (19 TR)) / 19, slot (P % (19 TR)) % 19
  long goff[NDW];
  int gst[NDW];
#pragma unroll
  for (int i = 0; i < NDW; ++i) {
    const int P = 64 * i + lane;
    const int sg = P / NPC, p = P - sg * NPC;
    const int tp = p / kWdPieces, j = p - tp * kWdPieces;
    const int tok = tp < tokens ? tp : tokens - 1;
    gst[i] = P < CPS * NPC ? sg : CPS;
    goff[i] = (long)tok * act_bytes + (j < 16 ? 4 + 16 * j : j == 16 ? 260 : j == 17 ? 276 : 0);
  }

  f32x16 acc[1][1];
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[0][0][e] = 0.0f;

  for (int base = sb0; base < sb1; base += CPS) {
    const int n = sb1 - base < CPS ? sb1 - base : CPS;
    if constexpr (TT == TT_Q6_K) {
      Q6Regs<true> wr[CPS];
#pragma unroll
      for (int s = 0; s < CPS; ++s) {
        if (s < n) {
          const uint8_t* b = wbase + (long)TILE * (base + s);
#pragma unroll
          for (int c = 0; c < 6; ++c) wr[s].p[c] = *(const u32x4*)(b + 1024 * c + 16 * lane);
          wr[s].sc = *(const u32x4*)(b + 6144 + 16 * li);
          wr[s].d = *(const uint16_t*)(b + 6656 + 2 * li);
        }
      }
#pragma unroll
      for (int i = 0; i < NDW; ++i)
        if (gst[i] < n)
          __builtin_amdgcn_global_load_lds((const void*)(XQ + goff[i] + 292L * (base + gst[i])),
                                           (__attribute__((address_space(3))) void*)(act + 1024 * i), 16, 0, 0);
      __builtin_amdgcn_s_waitcnt(0);  // this wave's weights and stages (no other wave reads them)
#pragma unroll
      for (int s = 0; s < CPS; ++s) {
        if (s < n) {
          const uint8_t* As = act + s * STAGE;
          QHIP_Q6K_SUPERBLOCK(wr[s], As, arow);
        }
      }
    } else {
      u32x4 wh[CPS], wq[CPS][4];
#pragma unroll
      for (int s = 0; s < CPS; ++s) {
        if (s < n) {
          const uint8_t* b = wbase + (long)TILE * (base + s);
          wh[s] = *(const u32x4*)(b + 4096 + 16 * li);
#pragma unroll
          for (int c = 0; c < 4; ++c) wq[s][c] = *(const u32x4*)(b + 1024 * c + 16 * lane);
        }
      }
#pragma unroll
      for (int i = 0; i < NDW; ++i)
        if (gst[i] < n)
          __builtin_amdgcn_global_load_lds((const void*)(XQ + goff[i] + 292L * (base + gst[i])),
                                           (__attribute__((address_space(3))) void*)(act + 1024 * i), 16, 0, 0);
      __builtin_amdgcn_s_waitcnt(0);  // this wave's weights and stages (no other wave reads them)
#pragma unroll
      for (int s = 0; s < CPS; ++s) {
        if (s < n) {
          const uint8_t* As = act + s * STAGE;
          QHIP_Q4K_SUPERBLOCK(wh[s], wq[s], As, arow);
        }
      }
    }
  }
  // the waves' partials, added in wave order
  __syncthreads();  // every wave is done with its stages
  float* red = (float*)lds;
#pragma unroll
  for (int e = 0; e < NE; ++e) red[(wv * NE + e) * 64 + lane] = acc[0][0][e];
  __syncthreads();
  if (wv == 0) {
    const int row = grp * 32 + li;
#pragma unroll
    for (int e = 0; e < NE; ++e) {
      float v = red[e * 64 + lane];
#pragma unroll
      for (int w = 1; w < NW; ++w) v += red[(w * NE + e) * 64 + lane];
      const int tok = 8 * (e >> 2) + 4 * lh + (e & 3);
      if (row < rows && tok < tokens) Y[(long)tok * rows + row] = v;
    }
  }
}

// Tokens per weights-direct tile: 32 up to 32 tokens (a 64-token tile would
// spend half its MFMA and epilogue work on padding) and from 65 to 96 (two
// 64-token tiles would pad up to 63 tokens; three 32-token ones pad at most
// 31), else 64.  Measured on MI355X, Q4_K from the image, weights from HBM,
// 65 / 80 / 96 tokens: [17408, 5120] 39.4 / 39.3 / 39.5 us against 45.0 /
// 45.3 / 45.8; [9728, 2560] 80 / 96 15.2 / 15.0 against 18.9 / 18.3;
// [12288, 4096] and [4096, 12288] at 96 26.7 / 27.6 against 29.0 / 28.7.
// 33 to 64 tokens keep one 64-token tile ([17408, 5120] 48 / 64 26.9 / 27.8
// us against 28.6 / 29.7 in two 32-token tiles), and 97 to 128 two
// ([9728, 2560] 128: 18.5 against 19.2).
static int wd_bt(const GemvArgs& g) { return g.tokens <= 32 || (g.tokens > 64 && g.tokens <= 96) ? 32 : 64; }

// K slices for a launch of one token tile (the few-token weights-direct and
// Q6_K kernels).  A workgroup's time is about its super-blocks times the time
// of one, and a super-block takes `share` times as long where two workgroups
// share a CU as where one runs alone (Q4_K about 1.6, Q6_K about 1.2); so the
// count minimises (super-blocks per slice) x (share if the grid has more
// workgroups than CUs, else 1), within one round of resident workgroups (two
// per CU) and with at
// least four super-blocks per slice (shorter slices never reach the copy
// pipeline's steady state), fewer slices on a tie.  Measured on MI355X, us
// (slices) against the earlier rule (aim at four workgroups per CU, two
// super-blocks per slice): Q4_K [17408, 5120] T = 32 / 48 / 64 20.7 / 27.4
// / 27.7 (3) against 22.5 / 34.6 / 35.1 (7) (2: 24.2 / 31.0 / 31.1, 4: 22.3
// / 32.2 / 32.8); [9728, 2560] T = 32 / 64 11.1 / 14.6 (3) against 12.8 /
// 17.5; [12288, 4096] 14.7 / 19.6 (4) against 17.2 / 25.5; [4096, 12288]
// 15.6 / 20.9 (8) against 23.2 / 34.1 (12: 16.7 / 23.9); [19456, 2560] T =
// 64 21.5 (3) against 25.6 (unsplit 20.2); Q6_K [5120, 17408] T = 20 / 32
// 28.2 / 30.9 (12) against 31.9 / 37.4 (23) (14: 31.9 / 40.1, 8: 34.6 /
// 38.1); [2560, 9728] 16.3 / 18.3 (10) against 17.1 / 19.1 (19); [4096,
// 12288] T = 24 / 32 21.3 / 23.1 (12) against 22.4 / 27.5 (24) (8: 23.9 /
// 25.8).
static int wd_one_round_slices(long tiles, int nsb, double share) {
  const int cus0 = qhip_gpu_cu_count(), cus = cus0 > 0 ? cus0 : 256;
  int best = 1;
  double best_c = (double)nsb * (tiles > cus ? share : 1.0);
  for (int s = 2; s <= nsb; ++s) {
    const int cps = (nsb + s - 1) / s, sl = (nsb + cps - 1) / cps;
    if (tiles * sl > 2L * cus || cps < 4) break;
    const double c = (double)cps * (tiles * sl > cus ? share : 1.0);
    if (c < best_c - 1e-9) {
      best_c = c;
      best = sl;
    }
  }
  return best;
}

// Grid plan of a weights-direct launch (wd_tile): the first nwhole tiles
// whole, the rest cut into ksplit slices.
struct WdPlan {
  int ksplit;
  long nwhole;
};

// With one token tile, every tile is cut into the one-round slice count
// (wd_one_round_slices).  With several
// token tiles and less than one round of resident workgroups (two per CU),
// every tile is cut by the round-filling count (mmq_round_slices).  From one
// round on, the whole rounds stay whole and only the tiles of the last,
// partial round are cut, into the slice count that minimises that round's
// cost in units of one whole tile: (rounds of slices) x (super-blocks per
// slice) / nsb, plus 0.13 per round of slices for their partial tiles'
// stores and loads; a partial round left whole costs 0.6 + 0.4 x its fill (a
// workgroup alone on its CU runs faster than two).
static WdPlan wd_plan(const GemvArgs& g) {
  const int nsb = g.cols / 256;
  const long ntt = (g.tokens + wd_bt(g) - 1) / wd_bt(g), tiles = ntt * ((g.rows + kWdBR - 1) / kWdBR);
  if (ntt < 2) return WdPlan{wd_one_round_slices(tiles, nsb, 1.6), 0};
  const int cus = qhip_gpu_cu_count();
  const long cap = 2L * (cus > 0 ? cus : 256);
  if (tiles < cap) return WdPlan{mmq_slices(nsb, mmq_round_slices(tiles, nsb, 2)), 0};
  const long rem = tiles % cap;
  WdPlan best{1, tiles};
  if (rem == 0 || rem > kSkMaxTiles) return best;
  double best_c = 0.6 + 0.4 * (double)rem / (double)cap;
  for (int cps = nsb / 2; cps >= 2; --cps) {
    const int sl = (nsb + cps - 1) / cps;
    if (sl < 2) continue;
    const long pieces = rem * sl, rounds = (pieces + cap - 1) / cap;
    const double c = (double)rounds * cps / nsb + 0.13 * (double)pieces / (double)cap;
    if (c < best_c - 1e-9) {
      best_c = c;
      best = WdPlan{sl, tiles - rem};
    }
  }
  return best;
}

static long wd_work_bytes(const GemvArgs& g, const WdPlan& p) {
  if (p.ksplit <= 1) return 0;
  const long tiles = ((g.tokens + wd_bt(g) - 1) / wd_bt(g)) * ((g.rows + kWdBR - 1) / kWdBR);
  return kSkCountBytes + 4L * p.ksplit * (tiles - p.nwhole) * wd_bt(g) * kWdBR;
}

template <bool IMG>
static hipError_t launch_mmq_wd(const GemvArgs& g, WdPlan plan, void* work, hipStream_t s, int bt) {
  const int nsb = g.cols / 256;
  const long ntt = (g.tokens + bt - 1) / bt, ntr = (g.rows + kWdBR - 1) / kWdBR, tiles = ntt * ntr;
  if (plan.ksplit <= 1) plan = WdPlan{1, tiles};
  const int ksplit = plan.ksplit;
  if (plan.nwhole < 0 || plan.nwhole > tiles) return hipErrorInvalidValue;
  const int cps = (nsb + ksplit - 1) / ksplit;
  const long nsplit = ksplit > 1 ? tiles - plan.nwhole : 0;
  const long G = ksplit > 1 ? plan.nwhole + nsplit * ksplit : tiles;
  if (G > 0x7FFFFFFFL || nsplit > kSkMaxTiles || (ksplit > 1 && (nsb + cps - 1) / cps != ksplit))
    return hipErrorInvalidValue;
  const int nwhole = (int)plan.nwhole;
  unsigned* cnt = ksplit > 1 ? (unsigned*)work : nullptr;
  float* part = ksplit > 1 ? (float*)((uint8_t*)work + kSkCountBytes) : nullptr;
  if constexpr (!IMG) {
    if (bt == 32 && g.tokens <= 24) {
      // few tokens: the raw-nibble form on the real tokens' elements (the
      // fragment image's few-token launches are k_mmq_rk)
      const int ng = (g.tokens + 7) / 8;
#define QHIP_WDS(N)                                                                                          \
  if (ng == N)                                                                                               \
    hipLaunchKernelGGL(k_mmq_wds_q4k<N>, dim3((unsigned)G), dim3(256), 0, s, (const uint8_t*)g.w,            \
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.row_bytes, g.act_bytes, nsb, ksplit, cps, \
                       part, cnt);
      QHIP_WDS(1) QHIP_WDS(2) QHIP_WDS(3)
#undef QHIP_WDS
      return hipGetLastError();
    }
  }
  if (bt == 32)
    hipLaunchKernelGGL((k_mmq_wd_q4k<1, IMG>), dim3((unsigned)G), dim3(256), 0, s, (const uint8_t*)g.w,
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.row_bytes, g.act_bytes, nsb, (int)ntt,
                       nwhole, ksplit, cps, part, cnt);
  else
    hipLaunchKernelGGL((k_mmq_wd_q4k<2, IMG>), dim3((unsigned)G), dim3(256), 0, s, (const uint8_t*)g.w,
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.row_bytes, g.act_bytes, nsb, (int)ntt,
                       nwhole, ksplit, cps, part, cnt);
  return hipGetLastError();
}

// Q6_K at up to 24 tokens on the default path: the few-token weights-direct
// kernel (one 32-token tile, 128 rows per workgroup, K split like the Q4_K one).
static bool wds_q6k(const GemvArgs& g) { return g.ttype == TT_Q6_K && g.tokens <= 24; }

// the tiles of every 32-token tile count: the fragment image's launch runs
// them side by side (blockIdx.y)
static int wds_q6k_slices(const GemvArgs& g) {
  const long ntt = (g.tokens + 31) / 32;
  return wd_one_round_slices(ntt * ((g.rows + kWdBR - 1) / kWdBR), g.cols / 256, 1.2);
}

static hipError_t launch_mmq_wds_q6k(const GemvArgs& g, int ksplit, void* work, hipStream_t s) {
  const int nsb = g.cols / 256;
  const long ntr = (g.rows + kWdBR - 1) / kWdBR;
  const int cps = (nsb + ksplit - 1) / ksplit;
  const long G = ntr * ksplit;
  if (G > 0x7FFFFFFFL || (ksplit > 1 && ntr > kSkMaxTiles)) return hipErrorInvalidValue;
  unsigned* cnt = ksplit > 1 ? (unsigned*)work : nullptr;
  float* part = ksplit > 1 ? (float*)((uint8_t*)work + kSkCountBytes) : nullptr;
  const int ng = (g.tokens + 7) / 8;
#define QHIP_WDS6(N)                                                                                          \
  if (ng == N)                                                                                                \
    hipLaunchKernelGGL(k_mmq_wds_q6k<N>, dim3((unsigned)G), dim3(256), 0, s, (const uint8_t*)g.w,             \
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.row_bytes, g.act_bytes, nsb, ksplit, cps, \
                       part, cnt);
  QHIP_WDS6(1) QHIP_WDS6(2) QHIP_WDS6(3)
#undef QHIP_WDS6
  return hipGetLastError();
}

// From the fragment image: Q6_K 1..32 tokens, Q4_K any count; work as for
// launch_mmq (the same slices as the GGUF-row launch, so mmq_work_bytes
// covers it).
template <int TT, int NW>
static hipError_t launch_mmq_rk(const GemvArgs& g, hipStream_t s) {
  const int nsb = g.cols / 256, ngrp = (g.rows + 31) / 32;
  const int cpw = (nsb + NW - 1) / NW;
  const int ng = (g.tokens + 7) / 8;
#define QHIP_RK(N)                                                                                               \
  if (ng == N)                                                                                                   \
    hipLaunchKernelGGL((k_mmq_rk<TT, N, NW, 1>), dim3((unsigned)ngrp), dim3(64 * NW), 0, s, (const uint8_t*)g.w, \
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.act_bytes, nsb, cpw);
  QHIP_RK(1) QHIP_RK(2) QHIP_RK(3)
#undef QHIP_RK
  return hipGetLastError();
}

long wd_image_work_bytes(const GemvArgs& g) {
  if (g.ttype == TT_Q4_K) return g.tokens <= 24 ? 0 : wd_work_bytes(g, wd_plan(g));
  if (g.ttype == TT_Q6_K && g.tokens > 16 && g.tokens <= 64) return mmq_split_bytes(g, 32, kWdBR, wds_q6k_slices(g));
  return 0;
}

hipError_t launch_mmq_wd_image(const GemvArgs& g, void* work, long work_bytes, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  if (g.ttype == TT_Q8_0) return launch_mmq_q8i(g, s);
  if (g.ttype == TT_Q4_K) {
    // up to 24 tokens the K split inside the workgroup; beyond, the 32- and
    // 64-token weights-direct tiles (split over workgroups on small grids)
    if (g.tokens <= 24) return launch_mmq_rk<TT_Q4_K, 4>(g, s);
    WdPlan plan = wd_plan(g);
    if (!work || work_bytes < wd_work_bytes(g, plan)) plan = WdPlan{1, 0};
    return launch_mmq_wd<true>(g, plan, work, s, wd_bt(g));
  }
  if (g.ttype != TT_Q6_K || g.tokens > 64) return hipErrorInvalidValue;
  // up to 16 tokens the K split inside the workgroup; 17..32 the split
  // launch with whole-group prefetch (28.0 against 28.3 us at 24 tokens)
  if (g.tokens <= 16) return launch_mmq_rk<TT_Q6_K, 12>(g, s);
  const int ntt = (g.tokens + 31) / 32;
  int ksplit = wds_q6k_slices(g);
  if (!work || work_bytes < mmq_split_bytes(g, 32, kWdBR, ksplit)) ksplit = 1;
  const int nsb = g.cols / 256;
  const long ntr = (g.rows + kWdBR - 1) / kWdBR;
  const int cps = (nsb + ksplit - 1) / ksplit;
  const long G = ntr * ksplit;
  if (G > 0x7FFFFFFFL || (ksplit > 1 && ntr * ntt > kSkMaxTiles)) return hipErrorInvalidValue;
  unsigned* cnt = ksplit > 1 ? (unsigned*)work : nullptr;
  float* part = ksplit > 1 ? (float*)((uint8_t*)work + kSkCountBytes) : nullptr;
  const int ng = ntt > 1 ? 4 : (g.tokens + 7) / 8;
#define QHIP_WDP(N)                                                                                           \
  if (ng == N)                                                                                                \
    hipLaunchKernelGGL((k_mmq_wdp_q6k<N, 2>), dim3((unsigned)G, (unsigned)ntt), dim3(256), 0, s, (const uint8_t*)g.w, \
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.act_bytes, nsb, ksplit, cps, part, cnt);
  QHIP_WDP(1) QHIP_WDP(2) QHIP_WDP(3) QHIP_WDP(4)
#undef QHIP_WDP
  return hipGetLastError();
}

// ---- launchers --------------------------------------------------------------------------
// `ksplit` is already the launched slice count (mmq_slices); work holds
// mmq_split_bytes when it is above 1
template <int TT, int BT, int BR, int NT = 256>
static hipError_t launch_mmq_t(const GemvArgs& g, int ksplit, void* work, hipStream_t s) {
  const int upr = g.cols / 64;
  const int nchunks = (upr + 3) / 4;
  const long ntr = (g.rows + BR - 1) / BR, ntt = (g.tokens + BT - 1) / BT;
  const int cps = (nchunks + ksplit - 1) / ksplit;
  const long G = ntr * ntt * ksplit;
  if (G > 0x7FFFFFFFL || (ksplit > 1 && ntr * ntt > kSkMaxTiles)) return hipErrorInvalidValue;
  unsigned* cnt = ksplit > 1 ? (unsigned*)work : nullptr;
  float* part = ksplit > 1 ? (float*)((uint8_t*)work + kSkCountBytes) : nullptr;
  if (ksplit > 1)
    hipLaunchKernelGGL((k_mmq<TT, BT, BR, NT, true>), dim3((unsigned)G), dim3(NT), 0, s, (const uint8_t*)g.w,
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.row_bytes, g.act_bytes, upr, (int)ntt,
                       ksplit, cps, part, cnt);
  else
    hipLaunchKernelGGL((k_mmq<TT, BT, BR, NT, false>), dim3((unsigned)G), dim3(NT), 0, s, (const uint8_t*)g.w,
                       (const uint8_t*)g.xq, g.out, g.rows, g.tokens, g.row_bytes, g.act_bytes, upr, (int)ntt,
                       ksplit, cps, part, cnt);
  return hipGetLastError();
}

template <int TT>
static hipError_t launch_mmq_type(const GemvArgs& g, int bt, int br, int ksplit, void* work, hipStream_t s) {
  // Q4_K's 64 x 128 tile is the weights-direct kernel (never split when
  // asked for explicitly)
  if constexpr (TT == TT_Q4_K)
    if (bt == 64 && br == 128)
      return launch_mmq_wd<false>(g, WdPlan{ksplit, 0}, work, s, g.tokens <= 32 ? 32 : 64);
  if (bt == 32 && br == 128) return launch_mmq_t<TT, 32, 128>(g, ksplit, work, s);
  if (bt == 32 && br == 64) return launch_mmq_t<TT, 32, 64, 128>(g, ksplit, work, s);
  if (bt == 64 && br == 64) return launch_mmq_t<TT, 64, 64>(g, ksplit, work, s);
  if (bt == 64 && br == 128) return launch_mmq_t<TT, 64, 128>(g, ksplit, work, s);
  if (bt == 128 && br == 64) return launch_mmq_t<TT, 128, 64>(g, ksplit, work, s);
  if (bt == 128 && br == 128) return launch_mmq_t<TT, 128, 128>(g, ksplit, work, s);
  return hipErrorInvalidValue;
}

// Default tile: 64 x 64 (Q4_K from 128 tokens: the weights-direct kernel
// above).  Measured on MI355X at the benchmark shapes (T = 16..512,
// all four formats) it beats the larger tiles everywhere: with one 32x32
// accumulator per wave it stays at 3-4 waves per SIMD, and the larger tiles'
// extra fragment reuse does not pay for their lower occupancy while the
// per-element scaling (VALU) is the bound.  K-quants with at most 32 tokens
// take one 32-token tile with the four waves stacked along 128 rows (a
// 64-token tile spends half its waves on padding): config 5 Q4_K at 16 tokens
// 23.5 vs 30.5 us, Q6_K 33.8 vs 42.9 us.  The 32-value formats keep 64 x 64:
// their (small) config-4 matrix needs the wider grid.
static void mmq_default_tile(const GemvArgs& g, int& bt, int& br) {
  const bool small = g.tokens <= 32 && !act32(g.ttype);
  bt = small ? 32 : 64;
  br = small ? 128 : 64;
  if (g.ttype == TT_Q4_K) {  // the weights-direct kernel
    bt = 64;
    br = 128;
  }
}


// Slices of the default tile launch.
static int mmq_default_slices(const GemvArgs& g, int bt, int br) {
  if (wds_q6k(g)) return wds_q6k_slices(g);
  const int nchunks = (g.cols / 64 + 3) / 4;
  return mmq_slices(nchunks, mmq_ksplit_for(g, bt, br, nchunks, 2));
}

long mmq_work_bytes(const GemvArgs& g) {
  int bt = 0, br = 0;
  mmq_default_tile(g, bt, br);
  if (g.ttype == TT_Q4_K && bt == 64 && br == 128) return wd_work_bytes(g, wd_plan(g));
  return mmq_split_bytes(g, bt, br, mmq_default_slices(g, bt, br));
}

hipError_t launch_mmq(const GemvArgs& g, int bt, int br, void* work, long work_bytes, hipStream_t s) {
  if (g.rows <= 0 || g.tokens <= 0) return hipSuccess;
  int ksplit = 1;
  if (bt <= 0 || br <= 0) {
    mmq_default_tile(g, bt, br);
    if (g.ttype == TT_Q4_K && bt == 64 && br == 128) {  // the weights-direct kernel
      WdPlan plan = wd_plan(g);
      if (!work || work_bytes < wd_work_bytes(g, plan)) plan = WdPlan{1, 0};
      return launch_mmq_wd<false>(g, plan, work, s, wd_bt(g));
    }
    ksplit = mmq_default_slices(g, bt, br);
    if (!work || work_bytes < mmq_split_bytes(g, bt, br, ksplit)) ksplit = 1;
    if (wds_q6k(g)) return launch_mmq_wds_q6k(g, ksplit, work, s);
  }
  switch (g.ttype) {
    case TT_Q8_0: return launch_mmq_type<TT_Q8_0>(g, bt, br, ksplit, work, s);
    case TT_IQ4_NL: return launch_mmq_type<TT_IQ4_NL>(g, bt, br, ksplit, work, s);
    case TT_Q4_0: return launch_mmq_type<TT_Q4_0>(g, bt, br, ksplit, work, s);
    case TT_Q4_1: return launch_mmq_type<TT_Q4_1>(g, bt, br, ksplit, work, s);
    case TT_IQ3_XXS: return launch_mmq_type<TT_IQ3_XXS>(g, bt, br, ksplit, work, s);
    case TT_IQ3_S: return launch_mmq_type<TT_IQ3_S>(g, bt, br, ksplit, work, s);
    case TT_Q4_K: return launch_mmq_type<TT_Q4_K>(g, bt, br, ksplit, work, s);
    case TT_Q6_K: return launch_mmq_type<TT_Q6_K>(g, bt, br, ksplit, work, s);
    case TT_Q5_K: return launch_mmq_type<TT_Q5_K>(g, bt, br, ksplit, work, s);
    case TT_IQ4_XS: return launch_mmq_type<TT_IQ4_XS>(g, bt, br, ksplit, work, s);
    case TT_Q3_K: return launch_mmq_type<TT_Q3_K>(g, bt, br, ksplit, work, s);
    case TT_Q2_K: return launch_mmq_type<TT_Q2_K>(g, bt, br, ksplit, work, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace qhip
