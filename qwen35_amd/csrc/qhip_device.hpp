// qhip_device.hpp -- device-side building blocks shared by the quantizer,
// GEMV and MMQ kernels: GGUF block geometry, exact f16 handling, int8 dot
// primitives, the IQ4_NL codebook lookup and the per-format decode of one
// 64-value work unit.
//
// The 32-value formats (Q8_0, IQ4_NL, Q4_0, Q4_1) pair with a Q8_0 activation
// (34 B / 32 values), the K-quants, IQ4_XS and the IQ3 grid formats with a
// Q8_K activation (292 B / 256 values), as the reference's actFamily
// (src/backend_cpu.zig:42-50) prescribes.
//
// Integer arithmetic inside a block is exact and equals the reference's
// per-block integers (src/kernels/x86/kernels32.c:342-361, :447-464;
// kernels256.c:474-498, :720-738); only the float folding of scaled block
// terms is reassociated.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq_grids.h"

#include <type_traits>

namespace qhip {

enum : int {
  TT_Q4_0 = 2, TT_Q4_1 = 3, TT_Q8_0 = 8, TT_Q2_K = 10, TT_Q3_K = 11, TT_Q4_K = 12, TT_Q5_K = 13,
  TT_Q6_K = 14, TT_IQ3_XXS = 18, TT_IQ4_NL = 20, TT_IQ3_S = 21, TT_IQ4_XS = 23
};

__host__ __device__ constexpr bool iq3(int tt) { return tt == TT_IQ3_XXS || tt == TT_IQ3_S; }

// Formats of 32-value blocks, which take a Q8_0 activation; the others take Q8_K.
__host__ __device__ constexpr bool act32(int tt) {
  return tt == TT_Q8_0 || tt == TT_IQ4_NL || tt == TT_Q4_0 || tt == TT_Q4_1;
}
// bytes of one 32-value weight block (act32 formats)
__host__ __device__ constexpr int blk32_bytes(int tt) {
  return tt == TT_Q8_0 ? 34 : tt == TT_Q4_1 ? 20 : 18;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2), aligned(4)));
// unaligned views (byte-aligned addresses; global memory only)
typedef uint32_t u32x4_u __attribute__((ext_vector_type(4), aligned(1)));
typedef uint32_t u32x2_u __attribute__((ext_vector_type(2), aligned(1)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));

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

// ---- activation quantizers, one block per lane group -------------------------------
// Q8_0 (src/kernels/x86/kernels32.c:1064-1087): lane i of a 32-lane group holds
// value i of the block.  Returns the lane's quantized value; `hbits` gets the
// block's f16 scale bits.  Every lane of the group must call it (shuffles).
__device__ __forceinline__ int quant_q8_0_lane(float v, uint32_t& hbits) {
  // |v| with the reference's "if (a > amax)" NaN handling: NaN never wins.
  float a = v < 0.0f ? -v : v;
  a = a > 0.0f ? a : 0.0f;
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
  const float scale = a > 0.0f ? a / 127.0f : 1.0f;
  const float inv = a > 0.0f ? 1.0f / scale : 0.0f;
  const float sv = v * inv;
  const float r = sv + (sv >= 0.0f ? 0.5f : -0.5f);
  int q = trunc_i32_x86(r);
  q = q > 127 ? 127 : q;
  q = q < -128 ? -128 : q;
  hbits = f32_to_f16_bits(scale);
  return q;
}

// Q8_K (src/kernels/x86/kernels256.c:865-896): lane l of a wave holds values
// 4l..4l+3 of the 256-value block.  Returns them quantized and packed (byte i
// = value 4l+i); `gsum` gets the sum of the lane's 16-value group (lanes 4g..4g+3
// agree), `scale` the block's f32 scale.  Every lane of the wave must call it.
__device__ __forceinline__ uint32_t quant_q8_K_lane(const float* v, int& gsum, float& scale) {
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float e = v[i] < 0.0f ? -v[i] : v[i];
    e = e > 0.0f ? e : 0.0f;
    a = fmaxf(a, e);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 64));
  scale = a > 0.0f ? a / 127.0f : 1.0f;
  const float inv = a > 0.0f ? 1.0f / scale : 0.0f;
  uint32_t packed = 0;
  int s = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float r = roundf(v[i] * inv);
    r = r < -127.0f ? -127.0f : r;
    r = r > 127.0f ? 127.0f : r;
    r = (r >= -127.0f) ? r : 127.0f;  // NaN
    const int q = (int)r;
    packed |= ((uint32_t)q & 0xFFu) << (8 * i);
    s += q;
  }
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  gsum = s;
  return packed;
}

// ---- wave reductions --------------------------------------------------------------
// Sum of v over the 64 lanes of a wave, in lane 63, by DPP (VALU lane moves:
// a few cycles each, against an LDS round trip per step for ds_bpermute).
// Adjacent lanes and lane pairs within quads (quad_perm), then the mirrored
// half-rows and rows give every lane of a 16-lane row the row's sum;
// row_bcast:15 adds row 0's sum into row 1 and row 2's into row 3,
// row_bcast:31 then adds rows 0 + 1 into rows 2 and 3.  The order of the
// additions is fixed, so the result is deterministic.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
  v += dpp_f32<0xB1>(v);         // quad_perm [1, 0, 3, 2]
  v += dpp_f32<0x4E>(v);         // quad_perm [2, 3, 0, 1]
  v += dpp_f32<0x141>(v);        // row_half_mirror
  v += dpp_f32<0x140>(v);        // row_mirror
  v += dpp_f32<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
  v += dpp_f32<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
  return v;
}

// ---- IQ4_NL codebook lookup on 4 packed indices --------------------------------
// Codebook (reference src/iq_tables.zig:429-432):
//   -127 -104 -83 -65 -49 -35 -22 -10 1 13 25 38 53 69 89 113
// v_perm_b32 selects bytes 0..7 of {src0:src1}.  Entries 0..7 and 8..15 are two
// 8-byte tables looked up with the low 3 index bits; a third perm then picks,
// per byte, the entry of the table that bit 3 names (selector byte i or 4+i).
constexpr uint32_t IQ4_T0 = 0xBFAD9881u;  // -127 -104  -83  -65
constexpr uint32_t IQ4_T1 = 0xF6EADDCFu;  //  -49  -35  -22  -10
constexpr uint32_t IQ4_T2 = 0x26190D01u;  //    1   13   25   38
constexpr uint32_t IQ4_T3 = 0x71594535u;  //   53   69   89  113

__device__ __forceinline__ uint32_t iq4_lookup(uint32_t s7, uint32_t pick) {
  const uint32_t lo = __builtin_amdgcn_perm(IQ4_T1, IQ4_T0, s7);
  const uint32_t hi = __builtin_amdgcn_perm(IQ4_T3, IQ4_T2, s7);
  return __builtin_amdgcn_perm(hi, lo, pick);
}
// Low / high nibbles of 4 packed bytes -> 4 int8 codebook values.
__device__ __forceinline__ uint32_t iq4_lo(uint32_t q) {
  return iq4_lookup(q & 0x07070707u, ((q >> 1) & 0x04040404u) | 0x03020100u);
}
__device__ __forceinline__ uint32_t iq4_hi(uint32_t q) {
  return iq4_lookup((q >> 4) & 0x07070707u, ((q >> 5) & 0x04040404u) | 0x03020100u);
}

// The integer dot of 8 packed indices against their activations, without the
// per-byte table select (for products that use each decoded weight once).
// v_perm_b32 with a selector byte of 8..15 reads no table entry: 8..11
// replicate the sign bit of table bytes 1, 3, 5, 7, 12 gives 0x00 and 13..15
// give 0xFF.  Each index n is looked up twice, in the low table with selector
// n (a codebook entry for n < 8) and in the high table with n ^ 8 (an entry
// for n >= 8); the other table's byte is then 0 or -1 as int8, and the tables
// hold the codebook plus 1 wherever the other side gives -1, so the two bytes
// always add up to the codebook value (L: low-table bytes 1, 3, 5, 7 are
// negative, so n = 8..11 read -1 from it; 13..15 read -1 from both; H:
// high-table bytes 1, 3, 5, 7 are positive, so n = 0..3 read 0 from it):
//   low  n = 0..7:  -127 -104 -83 -65 -49 -34 -21  -9   (codebook; 5..7 + 1)
//   high n = 8..15:    2   14  26  39  53  70  90 114   (codebook; 12 as is, others + 1)
// dot4 is linear, so the two bytes are multiplied separately: two perms and
// two dot4 per four values, and only the nibble masks and one xor besides.
constexpr uint32_t IQ4_L0 = 0xBFAD9881u;  // -127 -104  -83  -65
constexpr uint32_t IQ4_L1 = 0xF7EBDECFu;  //  -49  -34  -21   -9
constexpr uint32_t IQ4_H0 = 0x271A0E02u;  //    2   14   26   39
constexpr uint32_t IQ4_H1 = 0x725A4635u;  //   53   70   90  114

// byte j of q: low nibble -> the value multiplied by byte j of ya, high
// nibble -> byte j of yb
__device__ __forceinline__ int iq4_dot8(uint32_t q, uint32_t ya, uint32_t yb, int s) {
  const uint32_t nl = q & 0x0F0F0F0Fu, nh = (q >> 4) & 0x0F0F0F0Fu;
  s = dot4(__builtin_amdgcn_perm(IQ4_L1, IQ4_L0, nl), ya, s);
  s = dot4(__builtin_amdgcn_perm(IQ4_H1, IQ4_H0, nl ^ 0x08080808u), ya, s);
  s = dot4(__builtin_amdgcn_perm(IQ4_L1, IQ4_L0, nh), yb, s);
  s = dot4(__builtin_amdgcn_perm(IQ4_H1, IQ4_H0, nh ^ 0x08080808u), yb, s);
  return s;
}

// ---- IQ3 grids and signs --------------------------------------------------------
// The grids of iq_grids.h expanded to u32 entries (byte j = value j) in
// constant memory.  Kernels of an IQ3 format first stage their grid into LDS
// (grid_prologue), so the per-lane lookups are LDS reads, not divergent
// global loads; the byte-granular generic and dequant kernels read constant
// memory directly.
#define QHIP_XXS_ENTRY(c) QHIP_IQ3_EXPAND(QHIP_IQ3XXS_LEVEL, c),
#define QHIP_S_ENTRY(c) QHIP_IQ3_EXPAND(QHIP_IQ3S_LEVEL, c),
static __constant__ uint32_t kIq3xxsGrid[256] = {QHIP_IQ3XXS_CODES(QHIP_XXS_ENTRY)};
static __constant__ uint32_t kIq3sGrid[512] = {QHIP_IQ3S_CODES(QHIP_S_ENTRY)};
#undef QHIP_XXS_ENTRY
#undef QHIP_S_ENTRY
static __shared__ uint32_t g_iq3_grid[512];
// IQ3_XXS sign masks in LDS: entry s holds the parity-completed mask of the
// 7-bit index s as 0xFF / 0x00 bytes, .x for values 0..3, .y for 4..7 (one
// LDS read instead of the parity and byte spreading per 8 values; IQ3_S's
// explicit masks are spread in registers, which measured no slower).
static __shared__ uint2 g_iq3_sign[128];

// ksigns_iq2xs (src/iq_tables.zig:42-61): a 7-bit index completed by bit 7 to
// an even number of set bits; bit j negates value j of the 8.
__device__ __forceinline__ uint32_t iq_sign8(uint32_t idx7) {
  return idx7 | (((uint32_t)__builtin_popcount(idx7) & 1u) << 7);
}
// the low 4 bits of s as 0xFF / 0x00 bytes
__device__ __forceinline__ uint32_t sign_bytes4(uint32_t s) {
  const uint32_t t = ((s & 15u) * 0x00204081u) & 0x01010101u;
  return (t << 8) - t;
}

// ---- split-K hand-off between workgroups (deterministic) -----------------------
// The workgroups of one output tile each own a slice of K.  Each stores its
// partial sums with sk_store, then calls sk_arrive; the last workgroup of the
// tile to arrive (whichever it is) reads every slice's partials with sk_load,
// adds them in slice order -- so the result does not depend on which
// workgroup finished last -- and puts the tile's counter back to zero with
// sk_reset.  No workgroup waits for another.
//
// The guarantee this relies on, on gfx950 (LLVM AMDGPUUsage, memory model of
// the GFX942 family, which gfx950 follows):
//  * agent-scope atomic loads, stores and read-modify-writes are issued with
//    the sc1 cache-policy bit: stores are written through every XCD-private
//    cache to the agent coherence point, loads and RMWs are served from it,
//    never from a stale line of this XCD's L2 or the CU's L1;
//  * a store counts in vmcnt until the memory system acknowledges it, so after
//    `s_waitcnt vmcnt(0)` this wave's sc1 stores are performed at the
//    coherence point (an agent-scope release is `buffer_wbl2 sc1` followed by
//    exactly this wait; the write-back only matters for stores not already
//    written through, and every store the hand-off needs is an sc1 store);
//  * the workgroup barrier orders each wave's wait before thread 0's counter
//    RMW, and the last workgroup issues its sk_loads after the RMW that saw
//    the final count has returned (barrier again).
// So every partial is at the coherence point before the last workgroup's
// counter RMW can return the final count, and its sk_loads read them there.
// A release/acquire pair through __threadfence() gives the same order in
// terms of the HIP memory model, but writes back and invalidates the whole L2
// per workgroup: 25-490 us instead of about 10 us for the config-2 down
// projection (measured on MI355X).
__device__ __forceinline__ void sk_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float sk_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Every thread of the workgroup calls it after its sk_stores; true in every
// thread of the workgroup that brings the tile's count to `slices`.
__device__ __forceinline__ bool sk_arrive(unsigned* cnt, unsigned slices) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's partials are performed
  __syncthreads();
  __shared__ unsigned last;
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == slices - 1 ? 1u : 0u;
  __syncthreads();
  return last != 0;
}
// the last workgroup, once: the counter is zero again for the next launch
__device__ __forceinline__ void sk_reset(unsigned* cnt) {
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every thread of the workgroup must call it before any early exit.
template <int TT>
__device__ __forceinline__ void grid_prologue() {
  if constexpr (iq3(TT)) {
    constexpr int N = TT == TT_IQ3_XXS ? 256 : 512;
    for (int i = threadIdx.x; i < N; i += blockDim.x) g_iq3_grid[i] = TT == TT_IQ3_XXS ? kIq3xxsGrid[i] : kIq3sGrid[i];
    if constexpr (TT == TT_IQ3_XXS) {
      for (int i = threadIdx.x; i < 128; i += blockDim.x) {
        const uint32_t s8 = iq_sign8((uint32_t)i);
        g_iq3_sign[i] = make_uint2(sign_bytes4(s8), sign_bytes4(s8 >> 4));
      }
    }
    __syncthreads();
  }
}
// Four unsigned grid bytes (each >= 1) negated where the mask m is 0xFF:
// (g ^ m) + (m & 1) is 256 - g in those bytes, and no carry leaves a byte.
__device__ __forceinline__ uint32_t apply_mask4(uint32_t g, uint32_t m) { return (g ^ m) + (m & 0x01010101u); }

// ---- per-format unit decode ------------------------------------------------------
// Every GEMV lane walks a weight row in units of 64 values:
//   Q8_0    two 34-byte blocks (68 B, blocks 2u and 2u+1)
//   IQ4_NL  two 18-byte blocks (36 B); Q4_0 the same
//   Q4_1    two 20-byte blocks (40 B)
//   Q4_K    one quarter of a 144-byte super-block: 32 B of nibbles (sub-blocks
//           2c and 2c+1) plus the shared 16-byte header
//   Q6_K    one quarter of a 210-byte super-block: the (h, l-half) slice of the
//           ql/qh planes, four 16-value groups
// Consecutive units of a row are adjacent in memory.
//
// Each format gives
//   W, load_w(row, u)      weight registers of unit u, canonical (quants
//                          dword-aligned); `row` may point to global memory or
//                          to a copy of the row bytes in LDS
//   A, load_a(act, u)      activation registers of unit u from a quantized
//                          activation row in the reference layout (global)
//      load_a_split(sp, u) the same from the split layout in LDS (ActSplit)
//   ints(w, a, out)        the unit's exact integer partials
//   dot(w, a)              the unit's float contribution, built on ints()
// so the GEMV paths and the parity export share one integer core.
template <int TT>
struct Unit;

// Activation in LDS, split into planes (all 16-byte aligned):
//   qs  int8 values, 80 bytes per 64 (split_off)
//   d   per-block f32 scale (32-value blocks for Q8_0, 256 for Q8_K)
//   bs  Q8_K only: int16 sums of each 16 values
// Value v of the split image's int8 plane lives at byte split_off(v): 64-value
// units padded to 80 bytes, so the 16-byte reads of 16 lanes at consecutive
// units fall into distinct LDS banks (a 64-byte stride would put lanes j and
// j+4 on the same banks).
constexpr int kSplitUnit = 80;
__host__ __device__ constexpr int split_off(int v) { return (v >> 6) * kSplitUnit + (v & 63); }

struct ActSplit {
  const uint8_t* qs;
  const float* d;
  const int16_t* bs;
};

// 68-byte Q8_0 block pair (d0 q0[32] d1 q1[32]) at a 4-byte aligned address,
// canonicalised: q[0..7] block 0 quants, q[8..15] block 1 quants.
__device__ __forceinline__ void load_q8_pair(const uint8_t* p, uint32_t* q, uint32_t& d0, uint32_t& d1) {
  uint32_t v[17];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 x = ld128(p + 16 * i);
    v[4 * i] = x.x; v[4 * i + 1] = x.y; v[4 * i + 2] = x.z; v[4 * i + 3] = x.w;
  }
  v[16] = ld32(p + 64);
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = funnel(v[i + 1], v[i], 2);  // bytes 2..33
#pragma unroll
  for (int i = 0; i < 8; ++i) q[8 + i] = v[9 + i];                 // bytes 36..67
  d0 = v[0] & 0xFFFFu;
  d1 = v[8] >> 16;
}

// activation of a 32-value-block weight: two Q8_0 blocks (64 values)
struct ActPair {
  uint32_t q[16];
  float d0, d1;
};
__device__ __forceinline__ ActPair act_pair_ref(const uint8_t* act, int u) {
  ActPair a;
  uint32_t d0, d1;
  load_q8_pair(act + 68 * u, a.q, d0, d1);
  a.d0 = h2f(d0);
  a.d1 = h2f(d1);
  return a;
}
__device__ __forceinline__ ActPair act_pair_split(const ActSplit& sp, int u) {
  ActPair a;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u32x4 x = *(const u32x4*)(sp.qs + kSplitUnit * u + 16 * i);
    a.q[4 * i] = x.x; a.q[4 * i + 1] = x.y; a.q[4 * i + 2] = x.z; a.q[4 * i + 3] = x.w;
  }
  a.d0 = sp.d[2 * u];
  a.d1 = sp.d[2 * u + 1];
  return a;
}

template <>
struct Unit<TT_Q8_0> {
  static constexpr int kWBytes = 68, kInts = 2;
  struct W { uint32_t q[16]; uint32_t d0, d1; };
  using A = ActPair;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    W w;
    load_q8_pair(row + 68 * u, w.q, w.d0, w.d1);
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return act_pair_ref(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) { return act_pair_split(sp, u); }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* s) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s0 = dot4(w.q[i], a.q[i], s0);
      s1 = dot4(w.q[8 + i], a.q[8 + i], s1);
    }
    s[0] = s0;
    s[1] = s1;
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    return (h2f(w.d0) * a.d0) * (float)s[0] + (h2f(w.d1) * a.d1) * (float)s[1];
  }
};

template <>
struct Unit<TT_IQ4_NL> {
  static constexpr int kWBytes = 36, kInts = 2;
  struct W { uint32_t q[8]; uint32_t d0, d1; };  // q[0..3] block 0 indices, q[4..7] block 1
  using A = ActPair;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* p = row + 36 * u;
    uint32_t v[9];
    const u32x4 x0 = ld128(p), x1 = ld128(p + 16);
    v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
    v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    v[8] = ld32(p + 32);
    W w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w.q[i] = funnel(v[i + 1], v[i], 2);  // block 0 indices: bytes 2..17
      w.q[4 + i] = v[5 + i];               // block 1 indices: bytes 20..35
    }
    w.d0 = v[0] & 0xFFFFu;
    w.d1 = v[4] >> 16;
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return act_pair_ref(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) { return act_pair_split(sp, u); }
  // one block: 4 index dwords (byte j: low nibble -> value j, high nibble ->
  // value j+16) against 8 activation dwords (values 0..31)
  // (the select lookup here: with the GGUF rows' realigned loads it measured
  // faster than iq4_dot8, [248320, 2560] 71.3 against 77.0 us; IQ4_XS and the
  // GEMV image take iq4_dot8)
  static __device__ __forceinline__ int block(const uint32_t* q, const uint32_t* y) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s = dot4(iq4_lo(q[i]), y[i], s);
      s = dot4(iq4_hi(q[i]), y[4 + i], s);
    }
    return s;
  }
  static __device__ __forceinline__ int block_2t(const uint32_t* q, const uint32_t* y) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s = iq4_dot8(q[i], y[i], y[4 + i], s);
    return s;
  }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* s) {
    s[0] = block(w.q, a.q);
    s[1] = block(w.q + 4, a.q + 8);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    return (h2f(w.d0) * a.d0) * (float)s[0] + (h2f(w.d1) * a.d1) * (float)s[1];
  }
};

// 4 packed nibbles, one per byte (0..15) -> the int8 bytes nib - 8.  Setting
// bit 7 of every byte first keeps the per-byte subtraction from borrowing
// into its neighbour; flipping it back restores the two's complement byte.
__device__ __forceinline__ uint32_t nib_minus8(uint32_t n) {
  return ((n | 0x80808080u) - 0x08080808u) ^ 0x80808080u;
}

// Q4_0 (src/kernels/x86/kernels32.c:297-316): 18-byte blocks of f16 d and 16
// nibble bytes, byte j holding value j (low nibble) and j+16 (high), each
// value nib - 8.  The unit layout is IQ4_NL's.
template <>
struct Unit<TT_Q4_0> {
  static constexpr int kWBytes = 36, kInts = 2;
  using W = Unit<TT_IQ4_NL>::W;
  using A = ActPair;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) { return Unit<TT_IQ4_NL>::load_w(row, u); }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return act_pair_ref(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) { return act_pair_split(sp, u); }
  static __device__ __forceinline__ int block(const uint32_t* q, const uint32_t* y) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s = dot4(nib_minus8(q[i] & 0x0F0F0F0Fu), y[i], s);
      s = dot4(nib_minus8((q[i] >> 4) & 0x0F0F0F0Fu), y[4 + i], s);
    }
    return s;
  }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* s) {
    s[0] = block(w.q, a.q);
    s[1] = block(w.q + 4, a.q + 8);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    return (h2f(w.d0) * a.d0) * (float)s[0] + (h2f(w.d1) * a.d1) * (float)s[1];
  }
};

// Q4_1 (src/kernels/x86/kernels32.c:318-340): 20-byte blocks of f16 d, f16 m
// and 16 nibble bytes (unsigned values, same order as Q4_0); a block's term is
// d*dy*sumi + m*dy*sumy with sumy the sum of the activation block's int8s.
// A 40-byte unit of two blocks is dword aligned throughout: no funnel shifts.
template <>
struct Unit<TT_Q4_1> {
  static constexpr int kWBytes = 40, kInts = 4;
  struct W { uint32_t q[8]; uint32_t h0, h1; };  // h: d | m << 16
  using A = ActPair;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* p = row + 40 * u;
    const u32x4 x0 = ld128(p), x1 = ld128(p + 16);
    const u32x2 x2 = *(const u32x2*)(p + 32);
    W w;
    w.h0 = x0.x;
    w.q[0] = x0.y; w.q[1] = x0.z; w.q[2] = x0.w; w.q[3] = x1.x;
    w.h1 = x1.y;
    w.q[4] = x1.z; w.q[5] = x1.w; w.q[6] = x2.x; w.q[7] = x2.y;
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return act_pair_ref(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) { return act_pair_split(sp, u); }
  // (sumi, sumy) of one block; nibbles 0..15 are exact as signed int8
  static __device__ __forceinline__ void block(const uint32_t* q, const uint32_t* y, int& si, int& sy) {
    si = 0;
    sy = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      si = dot4(q[i] & 0x0F0F0F0Fu, y[i], si);
      si = dot4((q[i] >> 4) & 0x0F0F0F0Fu, y[4 + i], si);
      sy = dot4(0x01010101u, y[i], sy);
      sy = dot4(0x01010101u, y[4 + i], sy);
    }
  }
  // s = {sumi0, sumy0, sumi1, sumy1}
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* s) {
    block(w.q, a.q, s[0], s[1]);
    block(w.q + 4, a.q + 8, s[2], s[3]);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[4];
    ints(w, a, s);
    return (h2f(w.h0) * a.d0) * (float)s[0] + (h2f(w.h0 >> 16) * a.d0) * (float)s[1] +
           (h2f(w.h1) * a.d1) * (float)s[2] + (h2f(w.h1 >> 16) * a.d1) * (float)s[3];
  }
};

// activation of a K-quant quarter unit: 64 Q8_K values, the block scale and
// the four 16-value sums the unit needs
struct ActQ8K {
  uint32_t y[16];
  float d;
  int bs[4];
};

template <>
struct Unit<TT_Q4_K> {
  // unit u: super-block u>>2, quarter c = u&3 (values 64c..64c+63)
  static constexpr int kWBytes = 48, kInts = 2;
  struct W { uint32_t hdr[4]; uint32_t q[8]; int c; };
  using A = ActQ8K;
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
  // bsums of this quarter: groups 4c..4c+3
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
    const uint32_t b01 = ld32(blk + 260 + 8 * c), b23 = ld32(blk + 264 + 8 * c);
    a.bs[0] = sext16(b01); a.bs[1] = sext16(b01 >> 16);
    a.bs[2] = sext16(b23); a.bs[3] = sext16(b23 >> 16);
    return a;
  }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) {
    const int sb = u >> 2, c = u & 3;
    A a;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 x = *(const u32x4*)(sp.qs + kSplitUnit * (4 * sb + c) + 16 * i);
      a.y[4 * i] = x.x; a.y[4 * i + 1] = x.y; a.y[4 * i + 2] = x.z; a.y[4 * i + 3] = x.w;
    }
    a.d = sp.d[sb];
    const u32x2 b = *(const u32x2*)(sp.bs + 16 * sb + 4 * c);
    a.bs[0] = sext16(b.x); a.bs[1] = sext16(b.x >> 16);
    a.bs[2] = sext16(b.y); a.bs[3] = sext16(b.y >> 16);
    return a;
  }
  // isum over sub-blocks 2c (low nibbles) and 2c+1 (high nibbles); summs over
  // the bsums of those two sub-blocks.  The 6-bit scales and mins are unpacked
  // four at a time with the rule of src/kernels/x86/kernels256.c:105-125
  // applied bytewise, then the pair of this quarter is shifted out.
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) {
    int lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lo = dot4(w.q[i] & 0x0F0F0F0Fu, a.y[i], lo);
      hi = dot4((w.q[i] >> 4) & 0x0F0F0F0Fu, a.y[8 + i], hi);
    }
    const uint32_t S0 = w.hdr[1], S1 = w.hdr[2], S2 = w.hdr[3];
    const bool upper = w.c >= 2;  // sub-blocks 4..7
    const uint32_t scw = upper ? ((S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u)) : (S0 & 0x3F3F3F3Fu);
    const uint32_t mnw = upper ? (((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) : (S1 & 0x3F3F3F3Fu);
    const uint32_t sh = 16u * (uint32_t)(w.c & 1);
    const int sc0 = (int)((scw >> sh) & 0xFFu), sc1 = (int)((scw >> (sh + 8)) & 0xFFu);
    const int m0 = (int)((mnw >> sh) & 0xFFu), m1 = (int)((mnw >> (sh + 8)) & 0xFFu);
    out[0] = sc0 * lo + sc1 * hi;
    out[1] = m0 * (a.bs[0] + a.bs[1]) + m1 * (a.bs[2] + a.bs[3]);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    const float d = a.d * h2f(w.hdr[0]);
    const float dmin = a.d * h2f(w.hdr[0] >> 16);
    return d * (float)s[0] - dmin * (float)s[1];
  }
};

template <>
struct Unit<TT_Q6_K> {
  // unit u: super-block u>>2, h = (u>>1)&1, lh = u&1; values
  // 128h + 32q + 16lh + (0..15) for q = 0..3, in 16-value groups 8h + lh + 2q
  static constexpr int kWBytes = 52, kInts = 1;
  struct W { uint32_t la[4], lb[4], qh[4]; uint32_t sc01, sc23; uint32_t d; };
  using A = ActQ8K;
  // Q6_K super-blocks are 210 bytes, so every other one starts 2-byte
  // aligned.  gfx950 global loads take unaligned addresses (the target has
  // unaligned buffer access; the compiler emits one global_load_dwordx4 for
  // them), so each 16-byte piece is one load and every read stays inside the
  // super-block.
  static __device__ __forceinline__ void load16(const uint8_t* p, uint32_t* out) {
    const u32x4_u v = *(const u32x4_u*)p;
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  }
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 210 * (u >> 2);
    const int h = (u >> 1) & 1, lh = u & 1;
    W w;
    load16(blk + 64 * h + 16 * lh, w.la);
    load16(blk + 64 * h + 32 + 16 * lh, w.lb);
    load16(blk + 128 + 32 * h + 16 * lh, w.qh);
    // scales sc[8h + lh + 2q], q = 0..3: bytes 0, 2, 4, 6 of the 8 at ws
    const u32x2_u sc = *(const u32x2_u*)(blk + 192 + 8 * h + lh);
    w.sc01 = sc.x;
    w.sc23 = sc.y;
    w.d = *(const uint16_t*)(blk + 208);
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
    const int sh = 16 * lh;
    a.bs[0] = sext16(b.x >> sh); a.bs[1] = sext16(b.y >> sh);
    a.bs[2] = sext16(b.z >> sh); a.bs[3] = sext16(b.w >> sh);
    a.d = __builtin_bit_cast(float, ld32(blk));
    return a;
  }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) {
    const int sb = u >> 2, h = (u >> 1) & 1, lh = u & 1;
    A a;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 x = *(const u32x4*)(sp.qs + kSplitUnit * (4 * sb + 2 * h + (q >> 1)) + 32 * (q & 1) + 16 * lh);
      a.y[4 * q] = x.x; a.y[4 * q + 1] = x.y; a.y[4 * q + 2] = x.z; a.y[4 * q + 3] = x.w;
    }
    const u32x4 b = *(const u32x4*)(sp.bs + 16 * sb + 8 * h);
    const int sh = 16 * lh;
    a.bs[0] = sext16(b.x >> sh); a.bs[1] = sext16(b.y >> sh);
    a.bs[2] = sext16(b.z >> sh); a.bs[3] = sext16(b.w >> sh);
    a.d = sp.d[sb];
    return a;
  }
  // isum of the unit's four 16-value groups:
  //   sum_q sc[g] * sum_l (q6 - 32) * q8  =  sum_q sc[g] * (sum_l q6*q8 - 32*bsum[g])
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) {
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
    const int sc0 = sext8(w.sc01), sc1 = sext8(w.sc01 >> 16), sc2 = sext8(w.sc23), sc3 = sext8(w.sc23 >> 16);
    out[0] = sc0 * (s[0] - 32 * a.bs[0]) + sc1 * (s[1] - 32 * a.bs[1]) + sc2 * (s[2] - 32 * a.bs[2]) +
             sc3 * (s[3] - 32 * a.bs[3]);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[1];
    ints(w, a, s);
    return (h2f(w.d) * a.d) * (float)s[0];
  }
};

// ---- K-quant GEMV image (batch 1) ----
// Q4_K and Q6_K rows of a GEMV image hold the GGUF row's bytes, reordered so
// that lanes taking consecutive units load contiguous, aligned 16-byte
// pieces.  Units are grouped in chunks of 64 (the last chunk has m = U - 64c
// of the row's U units); piece e of unit 64c + i sits at 16 (NP 64c + m e + i),
// NP pieces per unit.  Q4_K (NP = 2: quant bytes 32q..32q+15 and
// 32q+16..32q+31 of quarter q = u & 3), then the 16-byte super-block headers
// (d, dmin, the 12 scale bytes) at 32 U + 16 sb.  Q6_K (NP = 3: the unit's
// 16 bytes of ql at 64h + 16lh, of ql at 64h + 32 + 16lh and of qh at
// 32h + 16lh), then each unit's four scales sc[8h + lh + 2q] at 48 U + 4u,
// then the super-blocks' f16 d at 52 U + 2 sb.  A row keeps its GGUF byte
// count, so row r of the image starts at r * row_bytes.
template <int TT>
struct KImg;

template <>
struct KImg<TT_Q4_K> {
  static constexpr int kPieces = 2;
  static __device__ __forceinline__ Unit<TT_Q4_K>::W load(const uint8_t* row, int u, int U) {
    const int c = u >> 6, i = u & 63, m = min(64, U - (c << 6));
    const uint8_t* p = row + 16L * (128 * c + i);
    Unit<TT_Q4_K>::W w;
    w.c = u & 3;
    const u32x4 a = ld128(p), b = ld128(p + 16 * m);
    const u32x4 h = ld128(row + 32L * U + 16 * (u >> 2));
    w.hdr[0] = h.x; w.hdr[1] = h.y; w.hdr[2] = h.z; w.hdr[3] = h.w;
    w.q[0] = a.x; w.q[1] = a.y; w.q[2] = a.z; w.q[3] = a.w;
    w.q[4] = b.x; w.q[5] = b.y; w.q[6] = b.z; w.q[7] = b.w;
    return w;
  }
};

template <>
struct KImg<TT_Q6_K> {
  static constexpr int kPieces = 3;
  static __device__ __forceinline__ Unit<TT_Q6_K>::W load(const uint8_t* row, int u, int U) {
    const int c = u >> 6, i = u & 63, m = min(64, U - (c << 6));
    const uint8_t* p = row + 16L * (192 * c + i);
    Unit<TT_Q6_K>::W w;
    // Q6_K rows are 210 bytes per super-block, so a row starts 2-byte aligned
    // at worst: unaligned loads (one global_load_dwordx4 each, as in the GGUF
    // path)
    const u32x4_u a = *(const u32x4_u*)p, b = *(const u32x4_u*)(p + 16 * m), q = *(const u32x4_u*)(p + 32 * m);
    const uint32_t sc = *(const u32_a2*)(row + 48L * U + 4 * u);
    w.la[0] = a.x; w.la[1] = a.y; w.la[2] = a.z; w.la[3] = a.w;
    w.lb[0] = b.x; w.lb[1] = b.y; w.lb[2] = b.z; w.lb[3] = b.w;
    w.qh[0] = q.x; w.qh[1] = q.y; w.qh[2] = q.z; w.qh[3] = q.w;
    // the dot reads bytes 0 and 2 of sc01 and sc23
    w.sc01 = (sc & 0xFFu) | ((sc & 0xFF00u) << 8);
    w.sc23 = ((sc >> 16) & 0xFFu) | ((sc >> 8) & 0xFF0000u);
    w.d = *(const uint16_t*)(row + 52L * U + 2 * (u >> 2));
    return w;
  }
};

// a unit's weights from the GGUF row or, IMG, from the K-quant image row
template <int TT, bool IMG>
__device__ __forceinline__ typename Unit<TT>::W load_unit(const uint8_t* row, int u, int U) {
  if constexpr (IMG) return KImg<TT>::load(row, u, U);
  else return Unit<TT>::load_w(row, u);
}

constexpr bool kimage_format(int tt) { return tt == TT_Q4_K || tt == TT_Q6_K; }


// ---- the further K-quant family (Q8_K activations, 64-value quarter units) ----
// Every unit below covers values 64c..64c+63 of super-block u>>2 (c = u&3) in
// order, so it takes the Q4_K activation unit (values, block scale, the four
// 16-value sums of groups 4c..4c+3).

template <>
struct Unit<TT_Q5_K> {
  // 176-byte super-block: d, dmin, 12 scale bytes, qh[32], qs[128]
  // (value layout src/kernels/x86/kernels256.c:188-198: nibble + 16 * bit)
  static constexpr int kWBytes = 80, kInts = 2;
  struct W { uint32_t hdr[4]; uint32_t q[8]; uint32_t qh[8]; int c; };
  using A = ActQ8K;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 176 * (u >> 2);
    W w;
    w.c = u & 3;
    const u32x4 h = ld128(blk), m0 = ld128(blk + 16), m1 = ld128(blk + 32);
    const u32x4 a = ld128(blk + 48 + 32 * w.c), b = ld128(blk + 64 + 32 * w.c);
    w.hdr[0] = h.x; w.hdr[1] = h.y; w.hdr[2] = h.z; w.hdr[3] = h.w;
    w.qh[0] = m0.x; w.qh[1] = m0.y; w.qh[2] = m0.z; w.qh[3] = m0.w;
    w.qh[4] = m1.x; w.qh[5] = m1.y; w.qh[6] = m1.z; w.qh[7] = m1.w;
    w.q[0] = a.x; w.q[1] = a.y; w.q[2] = a.z; w.q[3] = a.w;
    w.q[4] = b.x; w.q[5] = b.y; w.q[6] = b.z; w.q[7] = b.w;
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return Unit<TT_Q4_K>::load_a(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) {
    return Unit<TT_Q4_K>::load_a_split(sp, u);
  }
  // sub-blocks 2c (low nibbles, qh bit 2c) and 2c+1 (high nibbles, bit 2c+1);
  // scales and mins exactly as Q4_K (kernels256.c:605-629)
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) {
    int lo = 0, hi = 0;
    const uint32_t s0 = 2u * (uint32_t)w.c;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t h0 = ((w.qh[i] >> s0) & 0x01010101u) << 4;
      const uint32_t h1 = ((w.qh[i] >> (s0 + 1)) & 0x01010101u) << 4;
      lo = dot4((w.q[i] & 0x0F0F0F0Fu) | h0, a.y[i], lo);
      hi = dot4(((w.q[i] >> 4) & 0x0F0F0F0Fu) | h1, a.y[8 + i], hi);
    }
    const uint32_t S0 = w.hdr[1], S1 = w.hdr[2], S2 = w.hdr[3];
    const bool upper = w.c >= 2;
    const uint32_t scw = upper ? ((S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u)) : (S0 & 0x3F3F3F3Fu);
    const uint32_t mnw = upper ? (((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) : (S1 & 0x3F3F3F3Fu);
    const uint32_t sh = 16u * (uint32_t)(w.c & 1);
    const int sc0 = (int)((scw >> sh) & 0xFFu), sc1 = (int)((scw >> (sh + 8)) & 0xFFu);
    const int m0 = (int)((mnw >> sh) & 0xFFu), m1 = (int)((mnw >> (sh + 8)) & 0xFFu);
    out[0] = sc0 * lo + sc1 * hi;
    out[1] = m0 * (a.bs[0] + a.bs[1]) + m1 * (a.bs[2] + a.bs[3]);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    const float d = a.d * h2f(w.hdr[0]);
    const float dmin = a.d * h2f(w.hdr[0] >> 16);
    return d * (float)s[0] - dmin * (float)s[1];
  }
};

template <>
struct Unit<TT_Q3_K> {
  // 110-byte super-block: hmask[32], qs[64], 12 scale bytes, d.  Value
  // 128h + 32g + l = ((qs[32h+l] >> 2g) & 3) - (hmask bit 4h+g of byte l ? 0 : 4)
  // (kernels256.c:162-177).  Super-blocks start 2-byte aligned: unaligned
  // loads, each inside the super-block (see Unit<TT_Q6_K>).
  static constexpr int kWBytes = 78, kInts = 1;
  struct W { uint32_t q[8], hm[8]; uint32_t s0, s1, s2; uint32_t d; int c; };
  using A = ActQ8K;
  static __device__ __forceinline__ void load16(const uint8_t* p, uint32_t* out) {
    const u32x4_u v = *(const u32x4_u*)p;
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
  }
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 110 * (u >> 2);
    W w;
    w.c = u & 3;
    const int h = w.c >> 1;
    load16(blk, w.hm);
    load16(blk + 16, w.hm + 4);
    load16(blk + 32 + 32 * h, w.q);
    load16(blk + 48 + 32 * h, w.q + 4);
    const u32x2_u sc = *(const u32x2_u*)(blk + 96);
    w.s0 = sc.x;
    w.s1 = sc.y;
    w.s2 = *(const u32_a2*)(blk + 104);
    w.d = *(const uint16_t*)(blk + 108);
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return Unit<TT_Q4_K>::load_a(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) {
    return Unit<TT_Q4_K>::load_a_split(sp, u);
  }
  // groups 4c+k, k = 0..3: shift g = 2(c&1) + k/2, bytes 16(k&1).. of the qs
  // slice and of hmask.  sum (q3 - 4) * q8 = sum u3 * q8 - 4 * bsum with
  // u3 = q2 | (hbit << 2).  Scales: dword c of the 16 unpacked 6-bit values
  // (kernels256.c:129-151), used - 32.
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) {
    const int h = w.c >> 1;
    const uint32_t base = (w.c & 1) ? w.s1 : w.s0;
    const uint32_t scw = ((w.c >= 2 ? (base >> 4) : base) & 0x0F0F0F0Fu) |
                         (((w.s2 >> (2 * w.c)) & 0x03030303u) << 4);
    int isum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t g = 2u * (uint32_t)(w.c & 1) + (uint32_t)(k >> 1);
      const uint32_t hs = 4u * (uint32_t)h + g;
      int sk = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t q2 = (w.q[4 * (k & 1) + i] >> (2 * g)) & 0x03030303u;
        const uint32_t hb = (w.hm[4 * (k & 1) + i] >> hs) & 0x01010101u;
        sk = dot4(q2 | (hb << 2), a.y[4 * k + i], sk);
      }
      const int sc = (int)((scw >> (8 * k)) & 0xFFu) - 32;
      isum += sc * (sk - 4 * a.bs[k]);
    }
    out[0] = isum;
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[1];
    ints(w, a, s);
    return (h2f(w.d) * a.d) * (float)s[0];
  }
};

template <>
struct Unit<TT_Q2_K> {
  // 84-byte super-block: scales[16] (low nibble scale, high nibble min),
  // qs[64], d, dmin.  Value 128k + 32j + l = (qs[32k+l] >> 2j) & 3
  // (kernels256.c:153-160).
  static constexpr int kWBytes = 40, kInts = 2;
  struct W { uint32_t q[8]; uint32_t sc; uint32_t dd; int c; };
  using A = ActQ8K;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 84 * (u >> 2);
    W w;
    w.c = u & 3;
    const int k = w.c >> 1;
    const u32x4 a = ld128(blk + 16 + 32 * k), b = ld128(blk + 32 + 32 * k);
    w.q[0] = a.x; w.q[1] = a.y; w.q[2] = a.z; w.q[3] = a.w;
    w.q[4] = b.x; w.q[5] = b.y; w.q[6] = b.z; w.q[7] = b.w;
    w.sc = ld32(blk + 4 * w.c);
    w.dd = ld32(blk + 80);
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return Unit<TT_Q4_K>::load_a(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) {
    return Unit<TT_Q4_K>::load_a_split(sp, u);
  }
  // groups 4c+k: shift 2j with j = 2(c&1) + k/2, bytes 16(k&1).. of the slice
  // (kernels256.c:232-257)
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) {
    int isum = 0, summs = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t j = 2u * (uint32_t)(w.c & 1) + (uint32_t)(k >> 1);
      int sk = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) sk = dot4((w.q[4 * (k & 1) + i] >> (2 * j)) & 0x03030303u, a.y[4 * k + i], sk);
      const uint32_t b = (w.sc >> (8 * k)) & 0xFFu;
      isum += (int)(b & 15u) * sk;
      summs += (int)(b >> 4) * a.bs[k];
    }
    out[0] = isum;
    out[1] = summs;
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    const float dall = a.d * h2f(w.dd);
    const float dmin = a.d * h2f(w.dd >> 16);
    return dall * (float)s[0] - dmin * (float)s[1];
  }
};

template <>
struct Unit<TT_IQ4_XS> {
  // 136-byte super-block: d, scales_h (u16), scales_l[4], qs[128]; 32-value
  // block ib has index bytes qs[16ib..16ib+15] (low nibble -> value j, high ->
  // j+16) into the IQ4_NL codebook and the 6-bit scale
  // ls = scales_l nibble | 2 bits of scales_h, used - 32 (iq_kernels.c:967-1001)
  static constexpr int kWBytes = 40, kInts = 2;
  struct W { uint32_t q[8]; uint32_t h0, sl; int c; };
  using A = ActQ8K;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 136 * (u >> 2);
    W w;
    w.c = u & 3;
    const u32x4 a = ld128(blk + 8 + 32 * w.c), b = ld128(blk + 24 + 32 * w.c);
    w.q[0] = a.x; w.q[1] = a.y; w.q[2] = a.z; w.q[3] = a.w;
    w.q[4] = b.x; w.q[5] = b.y; w.q[6] = b.z; w.q[7] = b.w;
    w.h0 = ld32(blk);
    w.sl = ld32(blk + 4);
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return Unit<TT_Q4_K>::load_a(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) {
    return Unit<TT_Q4_K>::load_a_split(sp, u);
  }
  // the integers of blocks 2c and 2c+1, the IQ4_NL block core
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) {
    out[0] = Unit<TT_IQ4_NL>::block_2t(w.q, a.y);
    out[1] = Unit<TT_IQ4_NL>::block_2t(w.q + 4, a.y + 8);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    const uint32_t sh = w.h0 >> 16, sl = (w.sl >> (8 * w.c)) & 0xFFu;
    const int ls0 = (int)((sl & 15u) | (((sh >> (4 * w.c)) & 3u) << 4));
    const int ls1 = (int)((sl >> 4) | (((sh >> (4 * w.c + 2)) & 3u) << 4));
    const float d4d8 = h2f(w.h0) * a.d;
    return (d4d8 * (float)(ls0 - 32)) * (float)s[0] + (d4d8 * (float)(ls1 - 32)) * (float)s[1];
  }
};

// ---- IQ3 (Q8_K activations, quarter units as above) ------------------------------
template <>
struct Unit<TT_IQ3_XXS> {
  // 98-byte super-block: f16 d, qs[64] grid indices (one per 4 values), 8 u32
  // words (four 7-bit sign indices, the 4-bit scale in bits 28..31), one per
  // 32-value sub-block.  Unit c: indices qs[16c..16c+15], words 2c and 2c+1
  // (src/kernels/x86/iq_kernels.c:612-643).
  static constexpr int kWBytes = 26, kInts = 2;
  struct W { uint32_t q[4]; uint32_t aux[2]; uint32_t d; };
  using A = ActQ8K;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 98 * (u >> 2);
    const int c = u & 3;
    W w;
    const u32x4_u q = *(const u32x4_u*)(blk + 2 + 16 * c);
    w.q[0] = q.x; w.q[1] = q.y; w.q[2] = q.z; w.q[3] = q.w;
    const u32x2_u x = *(const u32x2_u*)(blk + 66 + 8 * c);
    w.aux[0] = x.x;
    w.aux[1] = x.y;
    w.d = *(const uint16_t*)blk;
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return Unit<TT_Q4_K>::load_a(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) {
    return Unit<TT_Q4_K>::load_a_split(sp, u);
  }
  // one 32-value sub-block: 8 index bytes q[0..1], its word, values y[0..7]
  static __device__ __forceinline__ int sub(const uint32_t* q, uint32_t aux, const uint32_t* y) {
    int s = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t qq = q[l >> 1] >> (16 * (l & 1));
      const uint2 m = g_iq3_sign[(aux >> (7 * l)) & 127u];
      s = dot4(apply_mask4(g_iq3_grid[qq & 255u], m.x), y[2 * l], s);
      s = dot4(apply_mask4(g_iq3_grid[(qq >> 8) & 255u], m.y), y[2 * l + 1], s);
    }
    return s;
  }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) {
    out[0] = sub(w.q, w.aux[0], a.y);
    out[1] = sub(w.q + 2, w.aux[1], a.y + 8);
  }
  // (d * dy) * sum (2 ls + 1) * sumi, times 1/4 (exact below 2^24)
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    const int ls0 = 2 * (int)(w.aux[0] >> 28) + 1, ls1 = 2 * (int)(w.aux[1] >> 28) + 1;
    return (h2f(w.d) * a.d) * (float)(ls0 * s[0] + ls1 * s[1]) * 0.25f;
  }
};

template <>
struct Unit<TT_IQ3_S> {
  // 110-byte super-block: f16 d, qs[64] low index bytes, qh[8] (bit k of
  // qh[ib] is index bit 8 of group k of sub-block ib), signs[32] (one mask per
  // 8 values), scales[4] (4-bit pairs).  Unit c: qs[16c..16c+15], qh[2c..2c+1],
  // signs[8c..8c+7], scales[c] (src/kernels/x86/iq_kernels.c:1728-1772).
  static constexpr int kWBytes = 30, kInts = 2;
  struct W { uint32_t q[4]; uint32_t sg[2]; uint32_t qh, sc, d; };
  using A = ActQ8K;
  static __device__ __forceinline__ W load_w(const uint8_t* row, int u) {
    const uint8_t* blk = row + 110 * (u >> 2);
    const int c = u & 3;
    W w;
    const u32x4_u q = *(const u32x4_u*)(blk + 2 + 16 * c);
    w.q[0] = q.x; w.q[1] = q.y; w.q[2] = q.z; w.q[3] = q.w;
    const u32x2_u s = *(const u32x2_u*)(blk + 74 + 8 * c);
    w.sg[0] = s.x;
    w.sg[1] = s.y;
    w.qh = *(const uint16_t*)(blk + 66 + 2 * c);
    w.sc = blk[106 + c];
    w.d = *(const uint16_t*)blk;
    return w;
  }
  static __device__ __forceinline__ A load_a(const uint8_t* act, int u) { return Unit<TT_Q4_K>::load_a(act, u); }
  static __device__ __forceinline__ A load_a_split(const ActSplit& sp, int u) {
    return Unit<TT_Q4_K>::load_a_split(sp, u);
  }
  static __device__ __forceinline__ uint32_t entry(uint32_t qq, uint32_t qh, int k) {
    return g_iq3_grid[(qq & 255u) | (((qh >> k) & 1u) << 8)];
  }
  // one 32-value sub-block: 8 low index bytes q[0..1], its qh byte, 4 sign masks
  static __device__ __forceinline__ int sub(const uint32_t* q, uint32_t qh, uint32_t sg, const uint32_t* y) {
    int s = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
      const uint32_t qq = q[l >> 1] >> (16 * (l & 1));
      const uint32_t s8 = sg >> (8 * l);
      s = dot4(apply_mask4(entry(qq, qh, 2 * l), sign_bytes4(s8)), y[2 * l], s);
      s = dot4(apply_mask4(entry(qq >> 8, qh, 2 * l + 1), sign_bytes4(s8 >> 4)), y[2 * l + 1], s);
    }
    return s;
  }
  static __device__ __forceinline__ void ints(const W& w, const A& a, int* out) {
    out[0] = sub(w.q, w.qh & 255u, w.sg[0], a.y);
    out[1] = sub(w.q + 2, w.qh >> 8, w.sg[1], a.y + 8);
  }
  static __device__ __forceinline__ float dot(const W& w, const A& a) {
    int s[2];
    ints(w, a, s);
    const int ls0 = 2 * (int)(w.sc & 15u) + 1, ls1 = 2 * (int)(w.sc >> 4) + 1;
    return (h2f(w.d) * a.d) * (float)(ls0 * s[0] + ls1 * s[1]);
  }
};

// Calls f(std::integral_constant<int, TT>{}) for the format id `ttype`.
template <class F>
__host__ inline auto dispatch_type(int ttype, F&& f) -> decltype(f(std::integral_constant<int, TT_Q8_0>{})) {
  switch (ttype) {
    case TT_Q8_0: return f(std::integral_constant<int, TT_Q8_0>{});
    case TT_IQ4_NL: return f(std::integral_constant<int, TT_IQ4_NL>{});
    case TT_Q4_K: return f(std::integral_constant<int, TT_Q4_K>{});
    case TT_Q6_K: return f(std::integral_constant<int, TT_Q6_K>{});
    case TT_Q5_K: return f(std::integral_constant<int, TT_Q5_K>{});
    case TT_Q3_K: return f(std::integral_constant<int, TT_Q3_K>{});
    case TT_Q2_K: return f(std::integral_constant<int, TT_Q2_K>{});
    case TT_IQ4_XS: return f(std::integral_constant<int, TT_IQ4_XS>{});
    case TT_Q4_0: return f(std::integral_constant<int, TT_Q4_0>{});
    case TT_Q4_1: return f(std::integral_constant<int, TT_Q4_1>{});
    case TT_IQ3_XXS: return f(std::integral_constant<int, TT_IQ3_XXS>{});
    case TT_IQ3_S: return f(std::integral_constant<int, TT_IQ3_S>{});
    default: return hipErrorInvalidValue;
  }
}


// ---- a weight unit decoded once, multiplied by several tokens --------------------
// The multi-token GEMV multiplies every weight unit it loads by up to eight
// tokens.  Prep<TT>::prep(w) does the unit's token-independent decode once
// (nibble and bit-plane unpacking, codebook lookups, scale unpacking, f16
// scale conversion) and Prep<TT>::dotp(p, a) is what is left per token: the
// dot4 products and the scaling, with the integers and the float expression of
// Unit<TT>::dot unchanged (same results bit for bit).  The default keeps the
// unit as loaded.
template <int TT>
struct Prep {
  using P = typename Unit<TT>::W;
  static __device__ __forceinline__ P prep(const typename Unit<TT>::W& w) { return w; }
  static __device__ __forceinline__ float dotp(const P& p, const typename Unit<TT>::A& a) { return Unit<TT>::dot(p, a); }
};

template <>
struct Prep<TT_Q4_K> {
  struct P { uint32_t lo[8], hi[8]; int sc0, sc1, m0, m1; float d, dmin; };
  static __device__ __forceinline__ P prep(const Unit<TT_Q4_K>::W& w) {
    P p;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p.lo[i] = w.q[i] & 0x0F0F0F0Fu;
      p.hi[i] = (w.q[i] >> 4) & 0x0F0F0F0Fu;
    }
    const uint32_t S0 = w.hdr[1], S1 = w.hdr[2], S2 = w.hdr[3];
    const bool upper = w.c >= 2;
    const uint32_t scw = upper ? ((S2 & 0x0F0F0F0Fu) | ((S0 >> 2) & 0x30303030u)) : (S0 & 0x3F3F3F3Fu);
    const uint32_t mnw = upper ? (((S2 >> 4) & 0x0F0F0F0Fu) | ((S1 >> 2) & 0x30303030u)) : (S1 & 0x3F3F3F3Fu);
    const uint32_t sh = 16u * (uint32_t)(w.c & 1);
    p.sc0 = (int)((scw >> sh) & 0xFFu);
    p.sc1 = (int)((scw >> (sh + 8)) & 0xFFu);
    p.m0 = (int)((mnw >> sh) & 0xFFu);
    p.m1 = (int)((mnw >> (sh + 8)) & 0xFFu);
    p.d = h2f(w.hdr[0]);
    p.dmin = h2f(w.hdr[0] >> 16);
    return p;
  }
  static __device__ __forceinline__ float dotp(const P& p, const ActQ8K& a) {
    int lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      lo = dot4(p.lo[i], a.y[i], lo);
      hi = dot4(p.hi[i], a.y[8 + i], hi);
    }
    const int isum = p.sc0 * lo + p.sc1 * hi;
    const int summs = p.m0 * (a.bs[0] + a.bs[1]) + p.m1 * (a.bs[2] + a.bs[3]);
    const float d = a.d * p.d;
    const float dmin = a.d * p.dmin;
    return d * (float)isum - dmin * (float)summs;
  }
};

template <>
struct Prep<TT_Q6_K> {
  struct P { uint32_t v[16]; int sc[4]; float d; };  // v[4q + i]: 0..63 values of group q
  static __device__ __forceinline__ P prep(const Unit<TT_Q6_K>::W& w) {
    P p;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t la = w.la[i], lb = w.lb[i], qh = w.qh[i];
      p.v[i] = (la & 0x0F0F0F0Fu) | ((qh & 0x03030303u) << 4);
      p.v[4 + i] = (lb & 0x0F0F0F0Fu) | ((qh << 2) & 0x30303030u);
      p.v[8 + i] = ((la >> 4) & 0x0F0F0F0Fu) | (qh & 0x30303030u);
      p.v[12 + i] = ((lb >> 4) & 0x0F0F0F0Fu) | ((qh >> 2) & 0x30303030u);
    }
    p.sc[0] = sext8(w.sc01);
    p.sc[1] = sext8(w.sc01 >> 16);
    p.sc[2] = sext8(w.sc23);
    p.sc[3] = sext8(w.sc23 >> 16);
    p.d = h2f(w.d);
    return p;
  }
  static __device__ __forceinline__ float dotp(const P& p, const ActQ8K& a) {
    int s[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q) s[q] = dot4(p.v[4 * q + i], a.y[4 * q + i], s[q]);
    const int isum = p.sc[0] * (s[0] - 32 * a.bs[0]) + p.sc[1] * (s[1] - 32 * a.bs[1]) +
                     p.sc[2] * (s[2] - 32 * a.bs[2]) + p.sc[3] * (s[3] - 32 * a.bs[3]);
    return (p.d * a.d) * (float)isum;
  }
};

template <>
struct Prep<TT_IQ4_NL> {
  struct P { uint32_t lo[8], hi[8]; float d0, d1; };  // [0..3] block 0, [4..7] block 1
  static __device__ __forceinline__ P prep(const Unit<TT_IQ4_NL>::W& w) {
    P p;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      p.lo[i] = iq4_lo(w.q[i]);
      p.hi[i] = iq4_hi(w.q[i]);
    }
    p.d0 = h2f(w.d0);
    p.d1 = h2f(w.d1);
    return p;
  }
  static __device__ __forceinline__ float dotp(const P& p, const ActPair& a) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s0 = dot4(p.lo[i], a.q[i], s0);
      s0 = dot4(p.hi[i], a.q[4 + i], s0);
      s1 = dot4(p.lo[4 + i], a.q[8 + i], s1);
      s1 = dot4(p.hi[4 + i], a.q[12 + i], s1);
    }
    return (p.d0 * a.d0) * (float)s0 + (p.d1 * a.d1) * (float)s1;
  }
};

}  // namespace qhip
