// qhip_device.hpp -- device-side building blocks shared by the quantizer,
// GEMV and MMQ kernels: GGUF block geometry, exact f16 handling, int8 dot
// primitives and the per-format decode of one 64-value work unit.
//
// Work unit.  Every kernel walks a weight row in units of 64 values:
//   Q8_0    two 34-byte blocks          (68 B, blocks 2u and 2u+1)
//   IQ4_NL  two 18-byte blocks          (36 B)
//   Q4_K    one quarter of a 144-byte super-block: 32 B of nibbles (sub-blocks
//           2c and 2c+1) plus the shared 16-byte header
//   Q6_K    one quarter of a 210-byte super-block: (h, l-half) of the
//           ql/qh planes, four 16-value groups
// Q8_0 and IQ4_NL pair with a Q8_0 activation (34 B / 32 values), Q4_K and
// Q6_K with a Q8_K activation (292 B / 256 values), as the reference's
// actFamily (src/backend_cpu.zig:42-50) prescribes.
//
// Integer arithmetic inside a block is exact and equals the reference's
// per-block integers (src/kernels/x86/kernels32.c:342-361, :447-464;
// kernels256.c:474-498, :720-738); only the float folding of scaled block
// terms is reassociated.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qhip {

enum : int { TT_Q8_0 = 8, TT_Q4_K = 12, TT_Q6_K = 14, TT_IQ4_NL = 20 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));

// ---- loads (addresses are 4-byte aligned; see each caller) -----------------
__device__ __forceinline__ uint32_t ld32(const uint8_t* p) { return *(const uint32_t*)p; }
__device__ __forceinline__ u32x4 ld128(const uint8_t* p) { return *(const u32x4*)p; }

// ---- int8 / byte primitives ---------------------------------------------------
__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
// bytes [sh, sh+4) of the 8-byte value {hi:lo}; sh in 0..3
__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, uint32_t sh) {
  return __builtin_amdgcn_alignbyte(hi, lo, sh);
}
// IEEE binary16 bits -> float.  v_cvt_f32_f16 is exact, subnormals included
// (the kernels run with f16 denormals preserved).
__device__ __forceinline__ float h2f(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}
__device__ __forceinline__ int sext16(uint32_t v) { return (int)(int16_t)(uint16_t)(v & 0xFFFFu); }
__device__ __forceinline__ int sext8(uint32_t v) { return (int)(int8_t)(uint8_t)(v & 0xFFu); }

// binary32 -> binary16 bits, round to nearest even, written with integer ops
// so no compiler conversion is involved.  Keeps the reference's quirks
// (src/kernels/x86/kernels32.c:67-98): NaN -> inf, and a value rounding up out
// of the subnormal range yields 0x0380.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t ex = (u >> 23) & 255u;
  const uint32_t mant = u & 0x7FFFFFu;
  if (ex >= 143u) return sign | 0x7C00u;  // >= 2^16, inf, nan
  if (ex >= 113u) {
    uint32_t m10 = mant >> 13;
    const uint32_t rest = mant & 0x1FFFu;
    m10 += (rest > 0x1000u || (rest == 0x1000u && (m10 & 1u))) ? 1u : 0u;
    uint32_t e16 = ex - 112u;
    if (m10 == 1024u) { m10 = 0; ++e16; }
    if (e16 >= 31u) return sign | 0x7C00u;
    return sign | (e16 << 10) | m10;
  }
  const int shift = 126 - (int)ex;  // 14..126
  if (shift >= 25) return sign;
  const uint32_t full = mant | 0x800000u;
  uint32_t m10 = full >> shift;
  const uint32_t rest = full & ((1u << shift) - 1u), half = 1u << (shift - 1);
  m10 += (rest > half || (rest == half && (m10 & 1u))) ? 1u : 0u;
  if (m10 >= 1024u) return sign | 0x0380u;
  return sign | m10;
}

// x86 cvttss2si semantics (truncate; INT_MIN for NaN or out of range), which
// is what the reference's (int) cast compiles to on its CPU path.
__device__ __forceinline__ int trunc_i32_x86(float v) {
  return (v > -2147483904.0f && v < 2147483648.0f) ? (int)v : (int)0x80000000u;
}

// ---- IQ4_NL codebook lookup on 4 packed indices --------------------------------
// Codebook (reference src/iq_tables.zig:429-432):
//   -127 -104 -83 -65 -49 -35 -22 -10 1 13 25 38 53 69 89 113
// v_perm_b32 selects bytes 0..7 of {src0:src1}; entries 0..7 and 8..15 are two
// 8-byte tables indexed by the low 3 bits, merged by bit 3 of each index.
constexpr uint32_t IQ4_T0 = 0xBFAD9881u;  // -127 -104  -83  -65
constexpr uint32_t IQ4_T1 = 0xF6EADDCFu;  //  -49  -35  -22  -10
constexpr uint32_t IQ4_T2 = 0x26190D01u;  //    1   13   25   38
constexpr uint32_t IQ4_T3 = 0x71594535u;  //   53   69   89  113

// sel: four indices in 0..7 (one per byte); bit3: per-byte 0x80 when the
// index is >= 8 (other bits ignored).
__device__ __forceinline__ uint32_t iq4_lut(uint32_t sel, uint32_t bit3) {
  const uint32_t lo = __builtin_amdgcn_perm(IQ4_T1, IQ4_T0, sel);
  const uint32_t hi = __builtin_amdgcn_perm(IQ4_T3, IQ4_T2, sel);
  // replicate bit 7 of every byte of bit3 across its byte
  const uint32_t m = (bit3 >> 7) & 0x01010101u;
  const uint32_t mask = (m << 8) - m;
  return (hi & mask) | (lo & ~mask);
}
// Low / high nibbles of 4 packed bytes -> 4 int8 codebook values.
__device__ __forceinline__ uint32_t iq4_lo(uint32_t q) { return iq4_lut(q & 0x07070707u, q << 4); }
__device__ __forceinline__ uint32_t iq4_hi(uint32_t q) { return iq4_lut((q >> 4) & 0x07070707u, q); }

// ---- Q4_K 6-bit scale / min of sub-block j (0..7) -------------------------------
// s0,s1,s2 are the 12 packed bytes (header bytes 4..15).  ggml's
// get_scale_min_k4 rule, equal to the reference unpack at
// src/kernels/x86/kernels256.c:105-125.
__device__ __forceinline__ void q4k_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                              int& sc, int& mn) {
  const uint32_t sh = 8u * (uint32_t)(j & 3);
  const uint32_t b0 = (s0 >> sh) & 0xFFu, b1 = (s1 >> sh) & 0xFFu, b2 = (s2 >> sh) & 0xFFu;
  if (j < 4) {
    sc = (int)(b0 & 63u);
    mn = (int)(b1 & 63u);
  } else {
    sc = (int)((b2 & 15u) | ((b0 >> 6) << 4));
    mn = (int)((b2 >> 4) | ((b1 >> 6) << 4));
  }
}

// ---- per-format unit decode ------------------------------------------------------
// Each format provides
//   W             weight registers of one unit
//   load_w        (row base, unit) -> W
//   A             activation registers of one unit
//   load_a        (activation row base, unit) -> A
//   dot           W x A -> float contribution (scaled, for GEMV)
//   ints          W x A -> exact integer partials of the unit (for parity)
template <int TT>
struct Unit;

template <>
struct Unit<TT_Q8_0> {
  static constexpr int kVals = 64, kWBytes = 68, kABytes = 68, kInts = 2;
  struct W { uint32_t v[17]; };
  struct A { uint32_t v[17]; };
  static __device__ __forceinline__ void load17(const uint8_t* p, uint32_t* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 x = ld128(p + 16 * i);
      v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
    }
    v[16] = ld32(p + 64);
  }
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    W w; load17(row + 68 * u, w.v); return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) {
    A a; load17(act + 68 * u, a.v); return a;
  }
  // Both sides share the 34-byte block layout, so byte k of the weight dword
  // pairs with byte k of the activation dword; the two scale bytes inside
  // dwords 0 and 8 are masked off on the weight side.
  static __device__ __forceinline__ void sums(const W& w, const A& a, int& s0, int& s1) {
    s0 = dot4(w.v[0] & 0xFFFF0000u, a.v[0], 0);
#pragma unroll
    for (int i = 1; i < 8; ++i) s0 = dot4(w.v[i], a.v[i], s0);
    s0 = dot4(w.v[8] & 0x0000FFFFu, a.v[8], s0);
    s1 = 0;
#pragma unroll
    for (int i = 9; i < 17; ++i) s1 = dot4(w.v[i], a.v[i], s1);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s0, s1;
    sums(w, a, s0, s1);
    const float d0 = h2f(w.v[0]) * h2f(a.v[0]);
    const float d1 = h2f(w.v[8] >> 16) * h2f(a.v[8] >> 16);
    return d0 * (float)s0 + d1 * (float)s1;
  }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) { sums(w, a, out[0], out[1]); }
};

template <>
struct Unit<TT_IQ4_NL> {
  static constexpr int kVals = 64, kWBytes = 36, kABytes = 68, kInts = 2;
  struct W { uint32_t v[9]; };
  using A = Unit<TT_Q8_0>::A;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* p = row + 36 * u;
    W w;
    const u32x4 x0 = ld128(p), x1 = ld128(p + 16);
    w.v[0] = x0.x; w.v[1] = x0.y; w.v[2] = x0.z; w.v[3] = x0.w;
    w.v[4] = x1.x; w.v[5] = x1.y; w.v[6] = x1.z; w.v[7] = x1.w;
    w.v[8] = ld32(p + 32);
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) {
    return Unit<TT_Q8_0>::load_a(act, u);
  }
  // One block: q[4] packed index bytes (byte j: low nibble -> value j, high
  // nibble -> value j+16), y[8] activation qs dwords (values 0..31).
  static __device__ __forceinline__ int block(const uint32_t* q, const uint32_t* y) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s = dot4(iq4_lo(q[i]), y[i], s);
      s = dot4(iq4_hi(q[i]), y[4 + i], s);
    }
    return s;
  }
  static __device__ __forceinline__ void sums(const W& w, const A& a, int& s0, int& s1) {
    uint32_t q0[4], q1[4], y0[8], y1[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      q0[i] = funnel(w.v[i + 1], w.v[i], 2);  // block 0 indices: bytes 2..17
      q1[i] = w.v[5 + i];                      // block 1 indices: bytes 20..35
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      y0[i] = funnel(a.v[i + 1], a.v[i], 2);  // activation block 0 qs: bytes 2..33
      y1[i] = a.v[9 + i];                      // activation block 1 qs: bytes 36..67
    }
    s0 = block(q0, y0);
    s1 = block(q1, y1);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s0, s1;
    sums(w, a, s0, s1);
    const float d0 = h2f(w.v[0]) * h2f(a.v[0]);
    const float d1 = h2f(w.v[4] >> 16) * h2f(a.v[8] >> 16);
    return d0 * (float)s0 + d1 * (float)s1;
  }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) { sums(w, a, out[0], out[1]); }
};

template <>
struct Unit<TT_Q4_K> {
  // unit u: super-block u>>2, quarter c = u&3 (values 64c..64c+63)
  static constexpr int kVals = 64, kWBytes = 48, kABytes = 64, kInts = 2;
  struct W { uint32_t hdr[4]; uint32_t q[8]; int c; };
  struct A { uint32_t y[16]; float d; uint32_t bs01, bs23; };
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 144 * (u >> 2);
    W w;
    w.c = u & 3;
    const u32x4 h = ld128(blk);
    const u32x4 a = ld128(blk + 16 + 32 * w.c), b = ld128(blk + 32 + 32 * w.c);
    w.hdr[0] = h.x; w.hdr[1] = h.y; w.hdr[2] = h.z; w.hdr[3] = h.w;
    w.q[0] = a.x; w.q[1] = a.y; w.q[2] = a.z; w.q[3] = a.w;
    w.q[4] = b.x; w.q[5] = b.y; w.q[6] = b.z; w.q[7] = b.w;
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) {
    const uint8_t* blk = act + 292 * (u >> 2);
    const int c = u & 3;
    A a;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 x = ld128(blk + 4 + 64 * c + 16 * i);
      a.y[4 * i] = x.x; a.y[4 * i + 1] = x.y; a.y[4 * i + 2] = x.z; a.y[4 * i + 3] = x.w;
    }
    a.d = __builtin_bit_cast(float, ld32(blk));
    a.bs01 = ld32(blk + 260 + 8 * c);
    a.bs23 = ld32(blk + 264 + 8 * c);
    return a;
  }
  // isum over sub-blocks 2c (low nibbles) and 2c+1 (high nibbles); summs over
  // the bsums of those two sub-blocks.
  static __device__ __forceinline__ void sums(const W& w, const A& a, int& isum, int& summs) {
    int lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lo = dot4(w.q[i] & 0x0F0F0F0Fu, a.y[i], lo);
      hi = dot4((w.q[i] >> 4) & 0x0F0F0F0Fu, a.y[8 + i], hi);
    }
    int sc0, m0, sc1, m1;
    q4k_scale_min(w.hdr[1], w.hdr[2], w.hdr[3], 2 * w.c, sc0, m0);
    q4k_scale_min(w.hdr[1], w.hdr[2], w.hdr[3], 2 * w.c + 1, sc1, m1);
    isum = sc0 * lo + sc1 * hi;
    summs = m0 * (sext16(a.bs01) + sext16(a.bs01 >> 16)) + m1 * (sext16(a.bs23) + sext16(a.bs23 >> 16));
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int isum, summs;
    sums(w, a, isum, summs);
    const float d = a.d * h2f(w.hdr[0]);
    const float dmin = a.d * h2f(w.hdr[0] >> 16);
    return d * (float)isum - dmin * (float)summs;
  }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) { sums(w, a, out[0], out[1]); }
};

template <>
struct Unit<TT_Q6_K> {
  // unit u: super-block u>>2, h = (u>>1)&1, lh = u&1; values 128h + 32q + 16lh + (0..15), q=0..3
  static constexpr int kVals = 64, kWBytes = 52, kABytes = 64, kInts = 1;
  struct W { uint32_t la[4], lb[4], qh[4]; uint32_t sc01, sc23; uint32_t d; };
  struct A { uint32_t y[16]; float d; uint32_t bs[4]; int lh; };
  // 16 bytes at a 2-byte aligned address: 5 aligned dwords, funnel-shifted.
  static __device__ __forceinline__ void load16(const uint8_t* p, uint32_t* out) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 3u;
    const uint8_t* b = p - sh;
    const u32x4 x = ld128(b);
    const uint32_t e = ld32(b + 16);
    out[0] = funnel(x.y, x.x, sh);
    out[1] = funnel(x.z, x.y, sh);
    out[2] = funnel(x.w, x.z, sh);
    out[3] = funnel(e, x.w, sh);
  }
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 210 * (u >> 2);
    const int h = (u >> 1) & 1, lh = u & 1;
    W w;
    load16(blk + 64 * h + 16 * lh, w.la);
    load16(blk + 64 * h + 32 + 16 * lh, w.lb);
    load16(blk + 128 + 32 * h + 16 * lh, w.qh);
    // scales sc[8h + lh + 2q], q = 0..3: bytes 0,2,4,6 of the window at ws
    const uint8_t* ws = blk + 192 + 8 * h + lh;
    const uint32_t ssh = (uint32_t)(uintptr_t)ws & 3u;
    const uint8_t* wb = ws - ssh;
    const uint32_t s0 = ld32(wb), s1 = ld32(wb + 4), s2 = ld32(wb + 8);
    w.sc01 = funnel(s1, s0, ssh);
    w.sc23 = funnel(s2, s1, ssh);
    const uint8_t* dp = blk + 208;
    const uint32_t dsh = (uint32_t)(uintptr_t)dp & 3u;
    w.d = ld32(dp - dsh) >> (8 * dsh);
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) {
    const uint8_t* blk = act + 292 * (u >> 2);
    const int h = (u >> 1) & 1, lh = u & 1;
    A a;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 x = ld128(blk + 4 + 128 * h + 32 * q + 16 * lh);
      a.y[4 * q] = x.x; a.y[4 * q + 1] = x.y; a.y[4 * q + 2] = x.z; a.y[4 * q + 3] = x.w;
    }
    const u32x4 b = ld128(blk + 260 + 16 * h);  // bsums of groups 8h..8h+7
    a.bs[0] = b.x; a.bs[1] = b.y; a.bs[2] = b.z; a.bs[3] = b.w;
    a.d = __builtin_bit_cast(float, ld32(blk));
    a.lh = lh;
    return a;
  }
  // isum of the unit's four 16-value groups g = 8h + lh + 2q:
  //   sum_q sc[g] * sum_l (q6 - 32) * q8  =  sum_q sc[g] * (sum_l q6*q8 - 32*bsum[g])
  static __device__ __forceinline__ int isum(const W& w, const A& a) {
    int s[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t la = w.la[i], lb = w.lb[i], qh = w.qh[i];
      const uint32_t v0 = (la & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4);
      const uint32_t v1 = (lb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
      const uint32_t v2 = ((la >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
      const uint32_t v3 = ((lb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
      s[0] = dot4(v0, a.y[i], s[0]);
      s[1] = dot4(v1, a.y[4 + i], s[1]);
      s[2] = dot4(v2, a.y[8 + i], s[2]);
      s[3] = dot4(v3, a.y[12 + i], s[3]);
    }
    const int sh = 16 * a.lh;
    const int sc0 = sext8(w.sc01), sc1 = sext8(w.sc01 >> 16), sc2 = sext8(w.sc23), sc3 = sext8(w.sc23 >> 16);
    const int b0 = sext16(a.bs[0] >> sh), b1 = sext16(a.bs[1] >> sh);
    const int b2 = sext16(a.bs[2] >> sh), b3 = sext16(a.bs[3] >> sh);
    return sc0 * (s[0] - 32 * b0) + sc1 * (s[1] - 32 * b1) + sc2 * (s[2] - 32 * b2) + sc3 * (s[3] - 32 * b3);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    return (h2f(w.d) * a.d) * (float)isum(w, a);
  }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) { out[0] = isum(w, a); }
};

}  // namespace qhip
