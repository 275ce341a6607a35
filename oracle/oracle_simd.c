/*
 * oracle_simd.c -- the host-ISA tiers of the CPU restatement (oracle.c), used
 * to time the reference's CPU path on the GPU box's host (bench.py's
 * cpu_baseline leg) at the speed the reference's own build would run it.
 *
 * TEST INFRASTRUCTURE ONLY (as oracle.c): the shipped HIP library never links
 * or calls it.  Each tier computes the same per-block integers as the scalar
 * restatement; the float fold follows the tier it restates:
 *
 *   IQ4_NL x Q8_0, AVX2   src/kernels/x86/kernels32.c:242-272: a 16-byte
 *                         codebook shuffle resolves 32 indices at once;
 *                         sequential per-block fold (bit-identical to scalar)
 *   Q8_0 x Q8_0, VNNI     src/kernels/x86/kernels512.c:53-81: i16-widened
 *                         pair products accumulated by vpdpwssd, reduced per
 *                         block; sequential fold (bit-identical to scalar)
 *   Q8_0 x Q8_0, AVX2     src/kernels/x86/kernels32.c:408-437: 8-lane FMA fold
 *   Q4_K x Q8_K, AVX2     src/kernels/x86/kernels256.c:500-599: u8 x s8 pair
 *                         sums scaled per sub-block in i32 lanes, one 8-lane
 *                         FMA per super-block, mins in a separate accumulator
 *   Q6_K x Q8_K, AVX2     src/kernels/x86/kernels256.c:740-859: 0..63 values
 *                         against s8, the -32 offset removed through the
 *                         activation's 16-value sums
 *
 * The tier is chosen at run time from the host's features, as the
 * reference's dispatch does (src/kernels/x86/cpu_caps.c:86-152,
 * src/simd_dispatch.zig:95-172).  Each function carries its own target
 * attribute, so this file builds without global ISA flags.
 */
#include "oracle.h"

#include <immintrin.h>
#include <stddef.h>
#include <string.h>

static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | ((unsigned)p[1] << 8)); }
static float rdf32(const uint8_t *p) { float f; memcpy(&f, p, 4); return f; }

#define AVX2 __attribute__((target("avx2,fma,f16c")))
#define VNNI __attribute__((target("avx512f,avx512bw,avx512vl,avx512vnni,avx2,fma")))

/* sum of 32 s8 x s8 products (|sum| <= 32*128*128 fits i32): the weight's
 * sign moved onto the activation so maddubs sees u8 x s8 */
AVX2 static inline __m256i pair_dot_s8(__m256i x, __m256i y) {
    const __m256i ax = _mm256_sign_epi8(x, x);
    const __m256i sy = _mm256_sign_epi8(y, x);
    return _mm256_madd_epi16(_mm256_maddubs_epi16(ax, sy), _mm256_set1_epi16(1));
}

AVX2 static inline int hsum_i32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xB1));
    return _mm_cvtsi128_si32(s);
}

AVX2 static inline float hsum_f32(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

/* kernels32.c:242-272 */
AVX2 static float dot_iq4_nl_avx2(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    const __m256i lut = _mm256_broadcastsi128_si256(_mm_loadu_si128((const __m128i *)kIq4nl));
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    float sumf = 0.0f;
    for (int b = 0; b < n / 32; ++b, w += 18, a += 34) {
        const float dw = orc_f16_to_f32(rd16(w)), da = orc_f16_to_f32(rd16(a));
        const __m128i q = _mm_loadu_si128((const __m128i *)(w + 2));
        /* low lane: low nibbles (values 0..15), high lane: high nibbles (16..31) */
        const __m256i idx = _mm256_and_si256(_mm256_set_m128i(_mm_srli_epi16(q, 4), q), m4);
        const __m256i wv = _mm256_shuffle_epi8(lut, idx);
        const __m256i av = _mm256_loadu_si256((const __m256i *)(a + 2));
        const int sumi = hsum_i32(pair_dot_s8(wv, av));
        sumf += dw * da * (float)sumi;
    }
    return sumf;
}

/* kernels32.c:408-437 */
AVX2 static float dot_q8_0_avx2(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < n / 32; ++b, w += 34, a += 34) {
        const float d = orc_f16_to_f32(rd16(w)) * orc_f16_to_f32(rd16(a));
        const __m256i wv = _mm256_loadu_si256((const __m256i *)(w + 2));
        const __m256i av = _mm256_loadu_si256((const __m256i *)(a + 2));
        const __m256i lo = _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm256_castsi256_si128(wv)),
                                             _mm256_cvtepi8_epi16(_mm256_castsi256_si128(av)));
        const __m256i hi = _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm256_extracti128_si256(wv, 1)),
                                             _mm256_cvtepi8_epi16(_mm256_extracti128_si256(av, 1)));
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(_mm256_add_epi32(lo, hi)), acc);
    }
    return hsum_f32(acc);
}

/* kernels512.c:53-81 */
VNNI static float dot_q8_0_vnni(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 32; ++b, w += 34, a += 34) {
        const float dw = orc_f16_to_f32(rd16(w)), da = orc_f16_to_f32(rd16(a));
        const __m512i wv = _mm512_cvtepi8_epi16(_mm256_loadu_si256((const __m256i *)(w + 2)));
        const __m512i av = _mm512_cvtepi8_epi16(_mm256_loadu_si256((const __m256i *)(a + 2)));
        const int sumi = _mm512_reduce_add_epi32(_mm512_dpwssd_epi32(_mm512_setzero_si512(), wv, av));
        sumf += dw * da * (float)sumi;
    }
    return sumf;
}

/* the eight 6-bit sub-block scales (out[0..7]) and mins (out[8..15]) of a
 * Q4_K header, kernels256.c:105-125 */
static void q4k_unpack(const uint8_t *s, uint8_t *out) {
    for (int j = 0; j < 4; ++j) {
        out[j] = s[j] & 63;
        out[8 + j] = s[j + 4] & 63;
        out[4 + j] = (uint8_t)((s[j + 8] & 15) | ((s[j] >> 6) << 4));
        out[12 + j] = (uint8_t)((s[j + 8] >> 4) | ((s[j + 4] >> 6) << 4));
    }
}

/* kernels256.c:500-599 */
AVX2 static float dot_q4_k_avx2(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    const __m256i m4 = _mm256_set1_epi8(0x0F);
    __m256 acc = _mm256_setzero_ps();
    __m128 acc_m = _mm_setzero_ps();
    for (int b = 0; b < n / 256; ++b, w += 144, a += 292) {
        const float dy = rdf32(a);
        const float d = dy * orc_f16_to_f32_k256(rd16(w));
        const float dmin = dy * orc_f16_to_f32_k256(rd16(w + 2));
        uint8_t sm[16];
        q4k_unpack(w + 4, sm);
        /* mins: pairs of 16-value sums against each sub-block's min */
        const __m256i bs = _mm256_loadu_si256((const __m256i *)(a + 260));
        const __m128i pair = _mm_hadd_epi16(_mm256_castsi256_si128(bs), _mm256_extracti128_si256(bs, 1));
        const __m128i mins = _mm_cvtepu8_epi16(_mm_loadl_epi64((const __m128i *)(sm + 8)));
        acc_m = _mm_fmadd_ps(_mm_set1_ps(-dmin), _mm_cvtepi32_ps(_mm_madd_epi16(mins, pair)), acc_m);
        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < 4; ++c) {
            const __m256i q = _mm256_loadu_si256((const __m256i *)(w + 16 + 32 * c));
            const __m256i lo = _mm256_and_si256(q, m4);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            const __m256i plo = _mm256_madd_epi16(_mm256_set1_epi16(sm[2 * c]),
                                                  _mm256_maddubs_epi16(lo, _mm256_loadu_si256((const __m256i *)(a + 4 + 64 * c))));
            const __m256i phi = _mm256_madd_epi16(_mm256_set1_epi16(sm[2 * c + 1]),
                                                  _mm256_maddubs_epi16(hi, _mm256_loadu_si256((const __m256i *)(a + 36 + 64 * c))));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(plo, phi));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    acc_m = _mm_add_ps(acc_m, _mm_movehl_ps(acc_m, acc_m));
    acc_m = _mm_add_ss(acc_m, _mm_movehdup_ps(acc_m));
    return hsum_f32(acc) + _mm_cvtss_f32(acc_m);
}

/* kernels256.c:740-859 */
AVX2 static float dot_q6_k_avx2(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    const __m256i m2 = _mm256_set1_epi8(3), m4 = _mm256_set1_epi8(15);
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < n / 256; ++b, w += 210, a += 292) {
        const float d = orc_f16_to_f32_k256(rd16(w + 208)) * rdf32(a);
        const int8_t *sc = (const int8_t *)(w + 192);
        /* 32 * sum_g sc[g] * bsum[g]: the -32 offset of every value */
        const __m256i bs = _mm256_loadu_si256((const __m256i *)(a + 260));
        const __m256i sc16 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)sc));
        const __m256 corr = _mm256_cvtepi32_ps(_mm256_slli_epi32(_mm256_madd_epi16(bs, sc16), 5));
        __m256i sumi = _mm256_setzero_si256();
        for (int h = 0; h < 2; ++h) {
            const __m256i qh = _mm256_loadu_si256((const __m256i *)(w + 128 + 32 * h));
            const __m256i qa = _mm256_loadu_si256((const __m256i *)(w + 64 * h));
            const __m256i qb = _mm256_loadu_si256((const __m256i *)(w + 64 * h + 32));
            __m256i v[4];
            v[0] = _mm256_or_si256(_mm256_and_si256(qa, m4), _mm256_slli_epi16(_mm256_and_si256(qh, m2), 4));
            v[1] = _mm256_or_si256(_mm256_and_si256(qb, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 2), m2), 4));
            v[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(qa, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 4), m2), 4));
            v[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(qb, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(qh, 6), m2), 4));
            for (int k = 0; k < 4; ++k) {
                /* 32 values = groups g, g+1: scale g on the low 128-bit half, g+1 on the high */
                const int g = 8 * h + 2 * k;
                const __m256i s = _mm256_set_m128i(_mm_set1_epi16(sc[g + 1]), _mm_set1_epi16(sc[g]));
                const __m256i q8 = _mm256_loadu_si256((const __m256i *)(a + 4 + 128 * h + 32 * k));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(s, _mm256_maddubs_epi16(v[k], q8)));
            }
        }
        const __m256 vd = _mm256_set1_ps(d);
        acc = _mm256_fmadd_ps(vd, _mm256_cvtepi32_ps(sumi), acc);
        acc = _mm256_fnmadd_ps(vd, corr, acc);
    }
    return hsum_f32(acc);
}

static int host_avx2(void) { return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma"); }
static int host_vnni(void) {
    return __builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") &&
           __builtin_cpu_supports("avx512vl") && __builtin_cpu_supports("avx512vnni");
}

orc_dot_fn orc_simd_dot_fn_for(int ttype) {
    if (ttype == ORC_TT_Q8_0 && host_vnni()) return dot_q8_0_vnni;
    if (!host_avx2()) return orc_dot_fn_for(ttype);
    switch (ttype) {
        case ORC_TT_Q8_0: return dot_q8_0_avx2;
        case ORC_TT_IQ4_NL: return dot_iq4_nl_avx2;
        case ORC_TT_Q4_K: return dot_q4_k_avx2;
        case ORC_TT_Q6_K: return dot_q6_k_avx2;
        default: return orc_dot_fn_for(ttype);
    }
}

/* the tier each type runs at on this host */
const char *orc_simd_tier(int ttype) {
    if (ttype == ORC_TT_Q8_0 && host_vnni()) return "avx512vnni";
    if (!host_avx2()) return "scalar";
    switch (ttype) {
        case ORC_TT_Q8_0: case ORC_TT_IQ4_NL: case ORC_TT_Q4_K: case ORC_TT_Q6_K: return "avx2";
        default: return "scalar";
    }
}

/* the AVX2 Q8_0 form even on a VNNI host (its fold differs: 8-lane FMA) */
orc_dot_fn orc_simd_dot_q8_0_avx2(void) { return host_avx2() ? dot_q8_0_avx2 : 0; }
