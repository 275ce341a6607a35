/*
 * oracle.c -- CPU restatement of the reference's quantized matvec arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker.  The shipped HIP library never
 * links or calls it.  Each function cites the reference file:line it follows
 * (paths relative to the reference repository).
 *
 * Built with -ffp-contract=off so every float expression rounds exactly as
 * written (no fused multiply-add), matching the reference's one-operation-
 * per-rounding statements.
 */
#include "oracle.h"
#include "../qwen35_amd/csrc/iq_grids.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* IQ4_NL codebook, reference src/iq_tables.zig:429-432 (ggml-common.h values). */
static const int8_t orc_iq4nl_values[16] = {
    -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113,
};

static uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | ((unsigned)p[1] << 8)); }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* IEEE binary16 -> binary32, exact; follows kernels32.c:45-66, including its
 * choice to return +0.0 for both signed zeros. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = ((uint32_t)h >> 10) & 31u;
    uint32_t mant = (uint32_t)h & 1023u;
    if (ex == 0) {
        if (mant == 0) return 0.0f;
        /* subnormal: shift the leading one up to bit 10 */
        int sh = 0;
        while (!(mant & 1024u)) { mant <<= 1; ++sh; }
        return bits_f32(sign | ((uint32_t)(113 - sh) << 23) | ((mant & 1023u) << 13));
    }
    if (ex == 31) return bits_f32(sign | 0x7F800000u | (mant << 13));
    return bits_f32(sign | ((ex + 112u) << 23) | (mant << 13));
}

/* Same decode as kernels256.c:51-78, which keeps the sign of zero. */
float orc_f16_to_f32_k256(uint16_t h) {
    if ((h & 0x7FFFu) == 0) return (h & 0x8000u) ? -0.0f : 0.0f;
    return orc_f16_to_f32(h);
}

/* binary32 -> binary16 bits, round to nearest even; follows kernels32.c:67-98.
 * Quirks kept on purpose because they are the reference's behaviour:
 *   NaN maps to infinity (sign kept);
 *   a value that rounds up out of the subnormal range (to 2^-14) yields the
 *   bit pattern 0x0380, not 0x0400 (kernels32.c:96). */
uint16_t orc_f32_to_f16(float x) {
    uint32_t u = f32_bits(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t ex = (u >> 23) & 255u;
    uint32_t mant = u & 0x7FFFFFu;
    if (ex == 255u || ex >= 143u) return (uint16_t)(sign | 0x7C00u);
    if (ex >= 113u) {
        uint32_t m10 = mant >> 13, rest = mant & 0x1FFFu;
        if (rest > 0x1000u || (rest == 0x1000u && (m10 & 1u))) ++m10;
        uint32_t e16 = ex - 112u;
        if (m10 == 1024u) { m10 = 0; ++e16; }
        if (e16 >= 31u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | (e16 << 10) | m10);
    }
    int shift = 126 - (int)ex; /* 14..126 */
    if (shift >= 25) return sign;
    uint32_t full = mant | 0x800000u;
    uint32_t m10 = full >> shift;
    uint32_t rest = full & ((1u << shift) - 1u), half = 1u << (shift - 1);
    if (rest > half || (rest == half && (m10 & 1u))) ++m10;
    if (m10 >= 1024u) return (uint16_t)(sign | 0x0380u);
    return (uint16_t)(sign | m10);
}

/* x86 cvttss2si: truncation, and INT_MIN for NaN / out-of-range.  The
 * reference's (int) casts run through it; stating it keeps non-finite inputs
 * defined here. */
static int32_t trunc_to_i32_x86(float v) {
    if (!(v > -2147483904.0f && v < 2147483648.0f)) return INT32_MIN;
    return (int32_t)v;
}

/* kernels32.c:1064-1087 */
void orc_quantize_q8_0(int n, const float *x, uint8_t *out) {
    for (int b = 0; b < n / 32; ++b) {
        const float *xb = x + 32 * b;
        uint8_t *ob = out + 34 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float a = xb[i] < 0.0f ? -xb[i] : xb[i];
            if (a > amax) amax = a;
        }
        float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        float inv = amax > 0.0f ? 1.0f / scale : 0.0f;
        uint16_t hb = orc_f32_to_f16(scale);
        ob[0] = (uint8_t)hb;
        ob[1] = (uint8_t)(hb >> 8);
        for (int i = 0; i < 32; ++i) {
            float v = xb[i] * inv;
            float r = v + (v >= 0.0f ? 0.5f : -0.5f);
            int32_t q = trunc_to_i32_x86(r);
            if (q > 127) q = 127;
            if (q < -128) q = -128;
            ob[2 + i] = (uint8_t)(int8_t)q;
        }
    }
}

/* kernels256.c:865-896 (clamp to [-127,127] per :886-888, NaN -> 127). */
void orc_quantize_q8_K(int n, const float *x, uint8_t *out) {
    for (int b = 0; b < n / 256; ++b) {
        const float *xb = x + 256 * b;
        uint8_t *ob = out + 292 * b;
        float amax = 0.0f;
        for (int i = 0; i < 256; ++i) {
            float a = xb[i] < 0.0f ? -xb[i] : xb[i];
            if (a > amax) amax = a;
        }
        float scale = amax > 0.0f ? amax / 127.0f : 1.0f;
        float inv = amax > 0.0f ? 1.0f / scale : 0.0f;
        memcpy(ob, &scale, 4);
        int16_t sums[16] = {0};
        for (int i = 0; i < 256; ++i) {
            float r = roundf(xb[i] * inv);
            if (r < -127.0f) r = -127.0f;
            if (r > 127.0f) r = 127.0f;
            if (!(r >= -127.0f)) r = 127.0f;
            int8_t q = (int8_t)(int32_t)r;
            ob[4 + i] = (uint8_t)q;
            sums[i / 16] = (int16_t)(sums[i / 16] + q);
        }
        memcpy(ob + 260, sums, 32);
    }
}

/* ---- exact per-block integers ------------------------------------------ */

/* kernels32.c:447-464: sum_j w[2+j]*a[2+j] over 32 int8 pairs. */
int32_t orc_blk_q8_0(const uint8_t *w, const uint8_t *a) {
    int32_t s = 0;
    for (int j = 0; j < 32; ++j) s += (int32_t)(int8_t)w[2 + j] * (int8_t)a[2 + j];
    return s;
}

/* kernels32.c:342-361: low nibble of qs[j] pairs with a[j], high with a[j+16]. */
int32_t orc_blk_iq4_nl(const uint8_t *w, const uint8_t *a) {
    int32_t s = 0;
    for (int j = 0; j < 16; ++j) {
        s += orc_iq4nl_values[w[2 + j] & 15] * (int32_t)(int8_t)a[2 + j];
        s += orc_iq4nl_values[w[2 + j] >> 4] * (int32_t)(int8_t)a[18 + j];
    }
    return s;
}

/* kernels32.c:297-316: Q4_0 block (f16 d @0, 16 nibble bytes @2); low
 * nibble of byte j minus 8 pairs with a[j], high nibble minus 8 with a[j+16]. */
int32_t orc_blk_q4_0(const uint8_t *w, const uint8_t *a) {
    int32_t s = 0;
    for (int j = 0; j < 16; ++j) {
        s += ((int32_t)(w[2 + j] & 15) - 8) * (int32_t)(int8_t)a[2 + j];
        s += ((int32_t)(w[2 + j] >> 4) - 8) * (int32_t)(int8_t)a[18 + j];
    }
    return s;
}

/* kernels32.c:318-340: Q4_1 block (f16 d @0, f16 m @2, 16 nibble bytes @4);
 * unsigned nibbles against a, and the sum of the block's 32 activations. */
void orc_blk_q4_1(const uint8_t *w, const uint8_t *a, int32_t *sumi, int32_t *sumy) {
    int32_t s = 0, y = 0;
    for (int j = 0; j < 16; ++j) {
        s += (int32_t)(w[4 + j] & 15) * (int32_t)(int8_t)a[2 + j];
        s += (int32_t)(w[4 + j] >> 4) * (int32_t)(int8_t)a[18 + j];
    }
    for (int j = 0; j < 32; ++j) y += (int32_t)(int8_t)a[2 + j];
    *sumi = s;
    *sumy = y;
}

/* 6-bit scale / min of sub-block sb (0..7) from the 12 packed bytes; the
 * ggml get_scale_min_k4 rule, equal to kernels256.c:105-125 (sm[sb] / sm[8+sb]). */
static void q4k_scale_min(const uint8_t *s12, int sb, int *sc, int *mn) {
    if (sb < 4) {
        *sc = s12[sb] & 63;
        *mn = s12[sb + 4] & 63;
    } else {
        *sc = (s12[sb + 4] & 15) | ((s12[sb - 4] >> 6) << 4);
        *mn = (s12[sb + 4] >> 4) | ((s12[sb] >> 6) << 4);
    }
}

/* kernels256.c:474-498 with :179-186 (nibble layout) and :216-226 (dot256):
 *   isum  = sum_g sc[g/2] * sum_{l<16} nib[16g+l] * q8[16g+l]
 *   summs = sum_{j<16} bsum[j] * min[j/2]                                   */
void orc_blk_q4_k(const uint8_t *w, const uint8_t *a, int32_t *isum, int32_t *summs) {
    const uint8_t *qs = w + 16;
    const int8_t *q8 = (const int8_t *)(a + 4);
    int32_t is = 0, sm = 0;
    for (int sb = 0; sb < 8; ++sb) {
        int sc, mn;
        q4k_scale_min(w + 4, sb, &sc, &mn);
        int c = sb / 2, hi = sb & 1;
        int32_t sub = 0;
        for (int l = 0; l < 32; ++l) {
            int nib = hi ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 15);
            sub += nib * (int32_t)q8[32 * sb + l];
        }
        is += sc * sub;
        for (int t = 0; t < 2; ++t) {
            int16_t bs;
            memcpy(&bs, a + 260 + 2 * (2 * sb + t), 2);
            sm += (int32_t)bs * mn;
        }
    }
    *isum = is;
    *summs = sm;
}

/* kernels256.c:200-212 (value layout) and :720-738:
 *   isum = sum_g sc[g] * sum_{l<16} (q6[16g+l] - 32) * q8[16g+l]              */
int32_t orc_blk_q6_k(const uint8_t *w, const uint8_t *a) {
    const uint8_t *ql = w, *qh = w + 128;
    const int8_t *sc = (const int8_t *)(w + 192);
    const int8_t *q8 = (const int8_t *)(a + 4);
    int32_t isum = 0;
    for (int g = 0; g < 16; ++g) {
        int32_t sub = 0;
        for (int l16 = 0; l16 < 16; ++l16) {
            int e = 16 * g + l16;
            int h = e / 128, q = (e % 128) / 32, l = e % 32;
            int lowbits = (q & 1) ? ql[64 * h + 32 + l] : ql[64 * h + l];
            lowbits = (q >= 2) ? (lowbits >> 4) : (lowbits & 15);
            int highbits = (qh[32 * h + l] >> (2 * q)) & 3;
            sub += ((lowbits | (highbits << 4)) - 32) * (int32_t)q8[e];
        }
        isum += sc[g] * sub;
    }
    return isum;
}

/* kernels256.c:605-629 with :188-198 (value layout: nibble + 16 * high bit)
 * and :216-226; scales/mins as Q4_K:
 *   isum  = sum_g sc[g/2] * sum_{l<16} q5[16g+l] * q8[16g+l]
 *   summs = sum_{j<16} bsum[j] * min[j/2]                                   */
void orc_blk_q5_k(const uint8_t *w, const uint8_t *a, int32_t *isum, int32_t *summs) {
    const uint8_t *qh = w + 16, *qs = w + 48;
    const int8_t *q8 = (const int8_t *)(a + 4);
    int32_t is = 0, sm = 0;
    for (int sb = 0; sb < 8; ++sb) {
        int sc, mn;
        q4k_scale_min(w + 4, sb, &sc, &mn);
        int c = sb / 2, hi = sb & 1;
        int32_t sub = 0;
        for (int l = 0; l < 32; ++l) {
            int v = hi ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 15);
            v += ((qh[l] >> sb) & 1) ? 16 : 0;
            sub += v * (int32_t)q8[32 * sb + l];
        }
        is += sc * sub;
        for (int t = 0; t < 2; ++t) {
            int16_t bs;
            memcpy(&bs, a + 260 + 2 * (2 * sb + t), 2);
            sm += (int32_t)bs * mn;
        }
    }
    *isum = is;
    *summs = sm;
}

/* Q3_K 6-bit scales, kernels256.c:129-151: sixteen values 0..63, used - 32. */
static void q3k_scales(const uint8_t *s12, int *sc) {
    uint32_t a0, a1, a2;
    memcpy(&a0, s12, 4);
    memcpy(&a1, s12 + 4, 4);
    memcpy(&a2, s12 + 8, 4);
    const uint32_t m1 = 0x03030303u, m2 = 0x0F0F0F0Fu;
    uint32_t u[4];
    u[0] = (a0 & m2) | (((a2 >> 0) & m1) << 4);
    u[1] = (a1 & m2) | (((a2 >> 2) & m1) << 4);
    u[2] = ((a0 >> 4) & m2) | (((a2 >> 4) & m1) << 4);
    u[3] = ((a1 >> 4) & m2) | (((a2 >> 6) & m1) << 4);
    for (int g = 0; g < 16; ++g) sc[g] = (int)((u[g / 4] >> (8 * (g % 4))) & 255u) - 32;
}

/* Q3_K value e = 128h + 32g + l: ((qs[32h+l] >> 2g) & 3) - (hmask bit 4h+g of
 * byte l ? 0 : 4), kernels256.c:162-177. */
static int q3k_value(const uint8_t *w, int e) {
    int h = e / 128, g = (e % 128) / 32, l = e % 32;
    int v = (w[32 + 32 * h + l] >> (2 * g)) & 3;
    return v - (((w[l] >> (4 * h + g)) & 1) ? 0 : 4);
}

/* kernels256.c:349-366: isum = sum_g (sc[g] - 32) * sum_{l<16} q3[16g+l] * q8[16g+l] */
int32_t orc_blk_q3_k(const uint8_t *w, const uint8_t *a) {
    const int8_t *q8 = (const int8_t *)(a + 4);
    int sc[16];
    q3k_scales(w + 96, sc);
    int32_t isum = 0;
    for (int g = 0; g < 16; ++g) {
        int32_t sub = 0;
        for (int l = 0; l < 16; ++l) sub += q3k_value(w, 16 * g + l) * (int32_t)q8[16 * g + l];
        isum += sc[g] * sub;
    }
    return isum;
}

/* kernels256.c:232-257 with :153-160 (value e = 128k + 32j + l:
 * (qs[32k+l] >> 2j) & 3):
 *   isum  = sum_g (scales[g] & 15) * sum_{l<16} q2[16g+l] * q8[16g+l]
 *   summs = sum_{j<16} bsum[j] * (scales[j] >> 4)                           */
void orc_blk_q2_k(const uint8_t *w, const uint8_t *a, int32_t *isum, int32_t *summs) {
    const int8_t *q8 = (const int8_t *)(a + 4);
    int32_t is = 0, sm = 0;
    for (int g = 0; g < 16; ++g) {
        int32_t sub = 0;
        for (int l16 = 0; l16 < 16; ++l16) {
            int e = 16 * g + l16;
            int k = e / 128, j = (e % 128) / 32, l = e % 32;
            sub += ((w[16 + 32 * k + l] >> (2 * j)) & 3) * (int32_t)q8[e];
        }
        is += (w[g] & 15) * sub;
        int16_t bs;
        memcpy(&bs, a + 260 + 2 * g, 2);
        sm += (int32_t)bs * (w[g] >> 4);
    }
    *isum = is;
    *summs = sm;
}

/* IQ4_XS 6-bit scale of 32-value block ib, iq_kernels.c:976-979: low nibble
 * from scales_l[ib/2], two high bits from scales_h. */
static int iq4xs_ls(const uint8_t *w, int ib) {
    int sh = ld16(w + 2);
    return ((w[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
}

/* iq_kernels.c:967-1001: the integer of 32-value block ib,
 *   sumi = sum_{j<16} q8[32ib+j] * kv[qs[16ib+j] & 15] + q8[32ib+16+j] * kv[qs[16ib+j] >> 4] */
int32_t orc_blk_iq4_xs(const uint8_t *w, const uint8_t *a, int ib) {
    const uint8_t *qs = w + 8 + 16 * ib;
    const int8_t *q8 = (const int8_t *)(a + 4) + 32 * ib;
    int32_t s = 0;
    for (int j = 0; j < 16; ++j)
        s += (int32_t)q8[j] * orc_iq4nl_values[qs[j] & 15] + (int32_t)q8[16 + j] * orc_iq4nl_values[qs[j] >> 4];
    return s;
}

/* ---- IQ3_XXS / IQ3_S ------------------------------------------------------
 * Grids: the 12-bit codes of iq_grids.h expanded to the u32 entries of
 * src/iq_tables.zig:323-356 / :360-425. */
#define ORC_XXS_ENTRY(c) QHIP_IQ3_EXPAND(QHIP_IQ3XXS_LEVEL, c),
#define ORC_S_ENTRY(c) QHIP_IQ3_EXPAND(QHIP_IQ3S_LEVEL, c),
static const uint32_t orc_iq3xxs_tab[256] = {QHIP_IQ3XXS_CODES(ORC_XXS_ENTRY)};
static const uint32_t orc_iq3s_tab[512] = {QHIP_IQ3S_CODES(ORC_S_ENTRY)};

uint32_t orc_iq3xxs_grid(int i) { return orc_iq3xxs_tab[i & 255]; }
uint32_t orc_iq3s_grid(int i) { return orc_iq3s_tab[i & 511]; }

/* ksigns_iq2xs (iq_tables.zig:42-61): the 7-bit index with bit 7 set when the
 * index has an odd number of ones, so every mask has even parity.  Bit j set
 * negates value j of the 8 (kmask_iq2xs, iq_tables.zig:36-38: 1 << j). */
uint8_t orc_ksigns(int i) {
    int p = 0;
    for (int b = 0; b < 7; ++b) p ^= (i >> b) & 1;
    return (uint8_t)((i & 127) | (p << 7));
}

/* 8 values: grid entries g1 (values 0..3), g2 (4..7) against q8, signs by mask */
static int32_t iq3_group(uint32_t g1, uint32_t g2, uint8_t sg, const int8_t *q8) {
    int32_t s = 0;
    for (int j = 0; j < 4; ++j) {
        s += (int32_t)((g1 >> (8 * j)) & 255) * q8[j] * ((sg >> j) & 1 ? -1 : 1);
        s += (int32_t)((g2 >> (8 * j)) & 255) * q8[4 + j] * ((sg >> (4 + j)) & 1 ? -1 : 1);
    }
    return s;
}

/* iq_kernels.c:612-643: sub-block ib of a 98-byte IQ3_XXS super-block (d,
 * qs[64] grid indices, 8 u32 aux words: four 7-bit sign indices, then the
 * 4-bit scale in bits 28..31) */
int32_t orc_blk_iq3_xxs(const uint8_t *w, const uint8_t *a, int ib) {
    const uint8_t *q3 = w + 2 + 8 * ib;
    uint32_t aux;
    memcpy(&aux, w + 66 + 4 * ib, 4);
    const int8_t *q8 = (const int8_t *)(a + 4) + 32 * ib;
    int32_t s = 0;
    for (int l = 0; l < 4; ++l)
        s += iq3_group(orc_iq3xxs_tab[q3[2 * l]], orc_iq3xxs_tab[q3[2 * l + 1]],
                       orc_ksigns((aux >> (7 * l)) & 127), q8 + 8 * l);
    return s;
}
static int iq3xxs_ls(const uint8_t *w, int ib) {
    uint32_t aux;
    memcpy(&aux, w + 66 + 4 * ib, 4);
    return 2 * (int)(aux >> 28) + 1;
}

/* iq_kernels.c:1728-1772: sub-block ib of a 110-byte IQ3_S super-block (d,
 * qs[64] low index bytes, qh[8] index bit 8, signs[32] explicit masks,
 * scales[4] 4-bit pairs); index of group k: qs[8ib+k] | bit k of qh[ib] << 8 */
int32_t orc_blk_iq3_s(const uint8_t *w, const uint8_t *a, int ib) {
    const uint8_t *qs = w + 2 + 8 * ib;
    const unsigned qh = w[66 + ib];
    const uint8_t *signs = w + 74 + 4 * ib;
    const int8_t *q8 = (const int8_t *)(a + 4) + 32 * ib;
    int32_t s = 0;
    for (int l = 0; l < 4; ++l) {
        const int i1 = qs[2 * l] | ((qh << (8 - 2 * l)) & 256);
        const int i2 = qs[2 * l + 1] | ((qh << (7 - 2 * l)) & 256);
        s += iq3_group(orc_iq3s_tab[i1], orc_iq3s_tab[i2], signs[l], q8 + 8 * l);
    }
    return s;
}
static int iq3s_ls(const uint8_t *w, int ib) { return 2 * ((w[106 + ib / 2] >> (4 * (ib % 2))) & 15) + 1; }

/* ---- geometry ------------------------------------------------------------ */

int orc_geom(int ttype, int *be, int *bb) {
    switch (ttype) {
    case ORC_TT_Q8_0: *be = 32; *bb = 34; return 1;
    case ORC_TT_IQ4_NL: *be = 32; *bb = 18; return 1;
    case ORC_TT_Q4_K: *be = 256; *bb = 144; return 1;
    case ORC_TT_Q6_K: *be = 256; *bb = 210; return 1;
    case ORC_TT_Q2_K: *be = 256; *bb = 84; return 1;
    case ORC_TT_Q3_K: *be = 256; *bb = 110; return 1;
    case ORC_TT_Q5_K: *be = 256; *bb = 176; return 1;
    case ORC_TT_IQ4_XS: *be = 256; *bb = 136; return 1;
    case ORC_TT_IQ3_XXS: *be = 256; *bb = 98; return 1;
    case ORC_TT_IQ3_S: *be = 256; *bb = 110; return 1;
    case ORC_TT_Q4_0: *be = 32; *bb = 18; return 1;
    case ORC_TT_Q4_1: *be = 32; *bb = 20; return 1;
    default: return 0;
    }
}

/* backend_cpu.zig:42-50 (actFamily): 32-element types take Q8_0, the rest Q8_K. */
int orc_act_block_elems(int ttype) {
    int be, bb;
    if (!orc_geom(ttype, &be, &bb)) return 0;
    return be == 32 ? 32 : 256;
}

long orc_act_bytes(int ttype, int cols) {
    int ab = orc_act_block_elems(ttype);
    if (!ab || cols <= 0 || cols % ab) return -1;
    return ab == 32 ? (long)cols / 32 * 34 : (long)cols / 256 * 292;
}

long orc_row_bytes(int ttype, int cols) {
    int be, bb;
    if (!orc_geom(ttype, &be, &bb) || cols <= 0 || cols % be) return -1;
    if (orc_act_bytes(ttype, cols) < 0) return -1;
    return (long)cols / be * bb;
}

/* ---- row dots ------------------------------------------------------------ */

static float dot_q8_0(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 32; ++b, w += 34, a += 34) {
        float dx = orc_f16_to_f32(ld16(w)), dy = orc_f16_to_f32(ld16(a));
        sumf += dx * dy * (float)orc_blk_q8_0(w, a);
    }
    return sumf;
}

static float dot_iq4_nl(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 32; ++b, w += 18, a += 34) {
        float dx = orc_f16_to_f32(ld16(w)), dy = orc_f16_to_f32(ld16(a));
        sumf += dx * dy * (float)orc_blk_iq4_nl(w, a);
    }
    return sumf;
}

/* kernels32.c:297-316, one sequential per-block fold (both tiers) */
static float dot_q4_0(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 32; ++b, w += 18, a += 34) {
        float dx = orc_f16_to_f32(ld16(w)), dy = orc_f16_to_f32(ld16(a));
        sumf += dx * dy * (float)orc_blk_q4_0(w, a);
    }
    return sumf;
}

/* kernels32.c:318-340: sumf += dx*dy*sumi + mx*dy*sumy per block */
static float dot_q4_1(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 32; ++b, w += 20, a += 34) {
        float dx = orc_f16_to_f32(ld16(w)), mx = orc_f16_to_f32(ld16(w + 2)), dy = orc_f16_to_f32(ld16(a));
        int32_t sumi, sumy;
        orc_blk_q4_1(w, a, &sumi, &sumy);
        sumf += dx * dy * (float)sumi + mx * dy * (float)sumy;
    }
    return sumf;
}

static float dot_q4_k(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 256; ++b, w += 144, a += 292) {
        int32_t isum, summs;
        orc_blk_q4_k(w, a, &isum, &summs);
        float dy;
        memcpy(&dy, a, 4);
        float d = dy * orc_f16_to_f32_k256(ld16(w));
        float dmin = dy * orc_f16_to_f32_k256(ld16(w + 2));
        sumf += d * (float)isum - dmin * (float)summs;
    }
    return sumf;
}

static float dot_q6_k(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 256; ++b, w += 210, a += 292) {
        float dy;
        memcpy(&dy, a, 4);
        sumf += orc_f16_to_f32_k256(ld16(w + 208)) * dy * (float)orc_blk_q6_k(w, a);
    }
    return sumf;
}

/* kernels256.c:605-629 */
static float dot_q5_k(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 256; ++b, w += 176, a += 292) {
        int32_t isum, summs;
        orc_blk_q5_k(w, a, &isum, &summs);
        float dy;
        memcpy(&dy, a, 4);
        float d = dy * orc_f16_to_f32_k256(ld16(w));
        float dmin = dy * orc_f16_to_f32_k256(ld16(w + 2));
        sumf += d * (float)isum - dmin * (float)summs;
    }
    return sumf;
}

/* kernels256.c:349-366 */
static float dot_q3_k(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 256; ++b, w += 110, a += 292) {
        float dy;
        memcpy(&dy, a, 4);
        sumf += orc_f16_to_f32_k256(ld16(w + 108)) * dy * (float)orc_blk_q3_k(w, a);
    }
    return sumf;
}

/* kernels256.c:232-257 */
static float dot_q2_k(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 256; ++b, w += 84, a += 292) {
        int32_t isum, summs;
        orc_blk_q2_k(w, a, &isum, &summs);
        float dy;
        memcpy(&dy, a, 4);
        float dall = dy * orc_f16_to_f32_k256(ld16(w + 80));
        float dmin = dy * orc_f16_to_f32_k256(ld16(w + 82));
        sumf += dall * (float)isum - dmin * (float)summs;
    }
    return sumf;
}

/* iq_kernels.c:967-1001 (the f16 decode at :163-196 keeps the sign of zero) */
static float dot_iq4_xs(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 256; ++b, w += 136, a += 292) {
        float dy;
        memcpy(&dy, a, 4);
        const float d4d8 = orc_f16_to_f32_k256(ld16(w)) * dy;
        for (int ib = 0; ib < 8; ++ib) {
            const float dl = d4d8 * (float)(iq4xs_ls(w, ib) - 32);
            sumf += dl * (float)orc_blk_iq4_xs(w, a, ib);
        }
    }
    return sumf;
}

/* iq_kernels.c:612-643: bsum = sum_ib sumi_ib * (2 ls + 1) per super-block,
 * sumf += (d * dy) * bsum, and 0.25 * sumf at the end */
static float dot_iq3_xxs(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 256; ++b, w += 98, a += 292) {
        float dy;
        memcpy(&dy, a, 4);
        const float d = orc_f16_to_f32_k256(ld16(w)) * dy;
        int32_t bsum = 0;
        for (int ib = 0; ib < 8; ++ib) bsum += orc_blk_iq3_xxs(w, a, ib) * iq3xxs_ls(w, ib);
        sumf += d * (float)bsum;
    }
    return 0.25f * sumf;
}

/* iq_kernels.c:1728-1772: as IQ3_XXS without the final 0.25 */
static float dot_iq3_s(int n, const void *vw, const void *va) {
    const uint8_t *w = vw, *a = va;
    float sumf = 0.0f;
    for (int b = 0; b < n / 256; ++b, w += 110, a += 292) {
        float dy;
        memcpy(&dy, a, 4);
        const float d = orc_f16_to_f32_k256(ld16(w)) * dy;
        int32_t bsum = 0;
        for (int ib = 0; ib < 8; ++ib) bsum += orc_blk_iq3_s(w, a, ib) * iq3s_ls(w, ib);
        sumf += d * (float)bsum;
    }
    return sumf;
}

orc_dot_fn orc_dot_fn_for(int ttype) {
    switch (ttype) {
    case ORC_TT_Q8_0: return dot_q8_0;
    case ORC_TT_IQ4_NL: return dot_iq4_nl;
    case ORC_TT_Q4_K: return dot_q4_k;
    case ORC_TT_Q6_K: return dot_q6_k;
    case ORC_TT_Q2_K: return dot_q2_k;
    case ORC_TT_Q3_K: return dot_q3_k;
    case ORC_TT_Q5_K: return dot_q5_k;
    case ORC_TT_IQ4_XS: return dot_iq4_xs;
    case ORC_TT_Q4_0: return dot_q4_0;
    case ORC_TT_Q4_1: return dot_q4_1;
    case ORC_TT_IQ3_XXS: return dot_iq3_xxs;
    case ORC_TT_IQ3_S: return dot_iq3_s;
    default: return 0;
    }
}

orc_quant_fn orc_quant_fn_for(int ttype) {
    int ab = orc_act_block_elems(ttype);
    return ab == 32 ? orc_quantize_q8_0 : ab == 256 ? orc_quantize_q8_K : 0;
}

float orc_dot(int ttype, int n, const void *w, const void *a) {
    orc_dot_fn f = orc_dot_fn_for(ttype);
    return f ? f(n, w, a) : NAN;
}

/* integers per weight block in orc_row_block_ints: (isum, summs) for the
 * K-quants with mins, (sumi, sumy) for Q4_1, one per 32-value block for
 * IQ4_XS and the IQ3 formats (before the block scales), else one */
int orc_block_nints(int ttype) {
    switch (ttype) {
    case ORC_TT_Q4_K: case ORC_TT_Q5_K: case ORC_TT_Q2_K: case ORC_TT_Q4_1: return 2;
    case ORC_TT_IQ4_XS: case ORC_TT_IQ3_XXS: case ORC_TT_IQ3_S: return 8;
    default: return 1;
    }
}

int orc_row_block_ints(int ttype, int n, const void *vw, const void *va, int32_t *out) {
    const uint8_t *w = vw, *a = va;
    int be, bb;
    if (!orc_geom(ttype, &be, &bb) || n % be) return -1;
    int nb = n / be;
    for (int b = 0; b < nb; ++b) {
        switch (ttype) {
        case ORC_TT_Q8_0: out[b] = orc_blk_q8_0(w + 34 * b, a + 34 * b); break;
        case ORC_TT_IQ4_NL: out[b] = orc_blk_iq4_nl(w + 18 * b, a + 34 * b); break;
        case ORC_TT_Q4_0: out[b] = orc_blk_q4_0(w + 18 * b, a + 34 * b); break;
        case ORC_TT_Q4_1: orc_blk_q4_1(w + 20 * b, a + 34 * b, &out[2 * b], &out[2 * b + 1]); break;
        case ORC_TT_Q4_K: orc_blk_q4_k(w + 144 * b, a + 292 * b, &out[2 * b], &out[2 * b + 1]); break;
        case ORC_TT_Q6_K: out[b] = orc_blk_q6_k(w + 210 * b, a + 292 * b); break;
        case ORC_TT_Q5_K: orc_blk_q5_k(w + 176 * b, a + 292 * b, &out[2 * b], &out[2 * b + 1]); break;
        case ORC_TT_Q2_K: orc_blk_q2_k(w + 84 * b, a + 292 * b, &out[2 * b], &out[2 * b + 1]); break;
        case ORC_TT_Q3_K: out[b] = orc_blk_q3_k(w + 110 * b, a + 292 * b); break;
        case ORC_TT_IQ4_XS:
            for (int ib = 0; ib < 8; ++ib) out[8 * b + ib] = orc_blk_iq4_xs(w + 136 * b, a + 292 * b, ib);
            break;
        case ORC_TT_IQ3_XXS:
            for (int ib = 0; ib < 8; ++ib) out[8 * b + ib] = orc_blk_iq3_xxs(w + 98 * b, a + 292 * b, ib);
            break;
        case ORC_TT_IQ3_S:
            for (int ib = 0; ib < 8; ++ib) out[8 * b + ib] = orc_blk_iq3_s(w + 110 * b, a + 292 * b, ib);
            break;
        }
    }
    return orc_block_nints(ttype) * nb;
}

int orc_quantize_act(int ttype, int cols, const float *x, uint8_t *out) {
    orc_quant_fn q = orc_quant_fn_for(ttype);
    if (!q || orc_act_bytes(ttype, cols) < 0) return -1;
    q(cols, x, out);
    return 0;
}

/* ---- matvec drivers ------------------------------------------------------ */

/* pool.zig:468-550 chunk rule: ~4 chunks per thread, clamped to [16, 256];
 * serial below 256 virtual rows (pool.zig:292-295). */
static int chunk_rows(long vrows, int nthreads) {
    long c = vrows / (4L * nthreads);
    if (c < 16) c = 16;
    if (c > 256) c = 256;
    return (int)c;
}

int orc_matvec_q_fn(orc_dot_fn dot, int ttype, int rows, int cols, int k,
                    const void *vw, const uint8_t *act, float *out, int nthreads) {
    long rb = orc_row_bytes(ttype, cols), ab = orc_act_bytes(ttype, cols);
    if (!dot || rb < 0 || ab < 0 || rows <= 0 || k <= 0) return -1;
    const uint8_t *w = vw;
    long vrows = (long)rows * k;
    if (nthreads < 1) nthreads = 1;
    if (nthreads == 1 || vrows < 256) {
        for (long r = 0; r < vrows; ++r) {
            long t = r / rows, rr = r % rows;
            out[t * rows + rr] = dot(cols, w + rr * rb, act + t * ab);
        }
        return 0;
    }
    int chunk = chunk_rows(vrows, nthreads);
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 1)
    for (long c0 = 0; c0 < vrows; c0 += chunk) {
        long c1 = c0 + chunk < vrows ? c0 + chunk : vrows;
        for (long r = c0; r < c1; ++r) {
            long t = r / rows, rr = r % rows;
            out[t * rows + rr] = dot(cols, w + rr * rb, act + t * ab);
        }
    }
    return 0;
}

int orc_matvec_batch_fn(orc_dot_fn dot, orc_quant_fn quant, int ttype, int rows,
                        int cols, int k, const void *w, const float *x, float *out,
                        uint8_t *act, int nthreads) {
    long ab = orc_act_bytes(ttype, cols);
    if (!quant || ab < 0 || k <= 0) return -1;
    for (int t = 0; t < k; ++t) quant(cols, x + (long)t * cols, act + t * ab);
    return orc_matvec_q_fn(dot, ttype, rows, cols, k, w, act, out, nthreads);
}

int orc_matvec_batch(int ttype, int rows, int cols, int k, const void *w,
                     const float *x, float *out, int nthreads) {
    long ab = orc_act_bytes(ttype, cols);
    if (ab < 0 || k <= 0) return -1;
    uint8_t *act = malloc((size_t)ab * k);
    if (!act) return -1;
    int rc = orc_matvec_batch_fn(orc_dot_fn_for(ttype), orc_quant_fn_for(ttype), ttype,
                                 rows, cols, k, w, x, out, act, nthreads);
    free(act);
    return rc;
}

/* ---- dequantization (fixture semantics) --------------------------------- */

/* quant_dequant.zig:1388-1402 (Q8_0), :347-360 (IQ4_NL), :78-103 (Q4_0,
 * Q4_1), :54-77 (Q4_K),
 * :222-251 (Q6_K), :188-220 (Q5_K), :252-322 (Q3_K), :892-919 (Q2_K),
 * :324-345 (IQ4_XS), :362-415 (IQ3_S), :417-445 (IQ3_XXS). */
int orc_dequant_row(int ttype, int cols, const void *vw, float *out) {
    const uint8_t *w = vw;
    if (orc_row_bytes(ttype, cols) < 0) return -1;
    if (ttype == ORC_TT_Q4_0 || ttype == ORC_TT_Q4_1) {
        const int bb = ttype == ORC_TT_Q4_0 ? 18 : 20, qo = ttype == ORC_TT_Q4_0 ? 2 : 4;
        for (int b = 0; b < cols / 32; ++b) {
            const uint8_t *blk = w + bb * b;
            float d = orc_f16_to_f32_k256(ld16(blk));
            float m = ttype == ORC_TT_Q4_1 ? orc_f16_to_f32_k256(ld16(blk + 2)) : 0.0f;
            for (int j = 0; j < 32; ++j) {
                int q = j < 16 ? (blk[qo + j] & 15) : (blk[qo + j - 16] >> 4);
                /* Q4_0: (q - 8) * d; Q4_1: q * d + m (two roundings) */
                out[32 * b + j] = ttype == ORC_TT_Q4_0 ? ((float)q - 8.0f) * d : (float)q * d + m;
            }
        }
        return 0;
    }
    if (ttype == ORC_TT_Q8_0 || ttype == ORC_TT_IQ4_NL) {
        int bb = ttype == ORC_TT_Q8_0 ? 34 : 18;
        for (int b = 0; b < cols / 32; ++b) {
            const uint8_t *blk = w + bb * b;
            /* quant_dequant.zig:34-37 converts with @floatCast, which keeps
             * the sign of a zero scale (unlike the dot path's k32 decode) */
            float d = orc_f16_to_f32_k256(ld16(blk));
            for (int j = 0; j < 32; ++j) {
                int v;
                if (ttype == ORC_TT_Q8_0) v = (int8_t)blk[2 + j];
                else v = orc_iq4nl_values[j < 16 ? (blk[2 + j] & 15) : (blk[2 + j - 16] >> 4)];
                out[32 * b + j] = d * (float)v;
            }
        }
        return 0;
    }
    for (int b = 0; b < cols / 256; ++b) {
        float *o = out + 256 * b;
        if (ttype == ORC_TT_Q4_K) {
            const uint8_t *blk = w + 144 * b;
            float d = orc_f16_to_f32_k256(ld16(blk)), mn = orc_f16_to_f32_k256(ld16(blk + 2));
            for (int sb = 0; sb < 8; ++sb) {
                int sc, m;
                q4k_scale_min(blk + 4, sb, &sc, &m);
                float d1 = d * (float)sc, m1 = mn * (float)m;
                for (int l = 0; l < 32; ++l) {
                    uint8_t q = blk[16 + 32 * (sb / 2) + l];
                    int nib = (sb & 1) ? (q >> 4) : (q & 15);
                    o[32 * sb + l] = d1 * (float)nib - m1;
                }
            }
        } else if (ttype == ORC_TT_Q5_K) {
            const uint8_t *blk = w + 176 * b;
            float d = orc_f16_to_f32_k256(ld16(blk)), mn = orc_f16_to_f32_k256(ld16(blk + 2));
            for (int sb = 0; sb < 8; ++sb) {
                int sc, m;
                q4k_scale_min(blk + 4, sb, &sc, &m);
                float d1 = d * (float)sc, m1 = mn * (float)m;
                for (int l = 0; l < 32; ++l) {
                    uint8_t q = blk[48 + 32 * (sb / 2) + l];
                    int v = ((sb & 1) ? (q >> 4) : (q & 15)) | (((blk[16 + l] >> sb) & 1) << 4);
                    o[32 * sb + l] = d1 * (float)v - m1;
                }
            }
        } else if (ttype == ORC_TT_Q3_K) {
            const uint8_t *blk = w + 110 * b;
            float d = orc_f16_to_f32_k256(ld16(blk + 108));
            int sc[16];
            q3k_scales(blk + 96, sc);
            for (int e = 0; e < 256; ++e) o[e] = (d * (float)sc[e / 16]) * (float)q3k_value(blk, e);
        } else if (ttype == ORC_TT_Q2_K) {
            const uint8_t *blk = w + 84 * b;
            float d = orc_f16_to_f32_k256(ld16(blk + 80)), mn = orc_f16_to_f32_k256(ld16(blk + 82));
            for (int e = 0; e < 256; ++e) {
                int g = e / 16, k = e / 128, j = (e % 128) / 32, l = e % 32;
                float dl = d * (float)(blk[g] & 15), ml = mn * (float)(blk[g] >> 4);
                o[e] = dl * (float)((blk[16 + 32 * k + l] >> (2 * j)) & 3) - ml;
            }
        } else if (ttype == ORC_TT_IQ3_XXS) {
            /* db = d * (0.5 + ls4) * 0.5; value = (db * g) * (+-1) */
            const uint8_t *blk = w + 98 * b;
            float d = orc_f16_to_f32_k256(ld16(blk));
            for (int ib = 0; ib < 8; ++ib) {
                uint32_t aux;
                memcpy(&aux, blk + 66 + 4 * ib, 4);
                const float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
                for (int l = 0; l < 4; ++l) {
                    const uint8_t sg = orc_ksigns((aux >> (7 * l)) & 127);
                    const uint32_t g1 = orc_iq3xxs_tab[blk[2 + 8 * ib + 2 * l]];
                    const uint32_t g2 = orc_iq3xxs_tab[blk[2 + 8 * ib + 2 * l + 1]];
                    for (int j = 0; j < 4; ++j) {
                        o[32 * ib + 8 * l + j] = db * (float)((g1 >> (8 * j)) & 255) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                        o[32 * ib + 8 * l + 4 + j] =
                            db * (float)((g2 >> (8 * j)) & 255) * ((sg >> (4 + j)) & 1 ? -1.0f : 1.0f);
                    }
                }
            }
        } else if (ttype == ORC_TT_IQ3_S) {
            /* db = d * (1 + 2 * nibble); value = (db * g) * (+-1) */
            const uint8_t *blk = w + 110 * b;
            float d = orc_f16_to_f32_k256(ld16(blk));
            for (int ib = 0; ib < 8; ++ib) {
                const float db = d * (float)iq3s_ls(blk, ib);
                const unsigned qh = blk[66 + ib];
                for (int l = 0; l < 4; ++l) {
                    const uint8_t sg = blk[74 + 4 * ib + l];
                    const uint32_t g1 = orc_iq3s_tab[blk[2 + 8 * ib + 2 * l] | ((qh << (8 - 2 * l)) & 256)];
                    const uint32_t g2 = orc_iq3s_tab[blk[2 + 8 * ib + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256)];
                    for (int j = 0; j < 4; ++j) {
                        o[32 * ib + 8 * l + j] = db * (float)((g1 >> (8 * j)) & 255) * ((sg >> j) & 1 ? -1.0f : 1.0f);
                        o[32 * ib + 8 * l + 4 + j] =
                            db * (float)((g2 >> (8 * j)) & 255) * ((sg >> (4 + j)) & 1 ? -1.0f : 1.0f);
                    }
                }
            }
        } else if (ttype == ORC_TT_IQ4_XS) {
            const uint8_t *blk = w + 136 * b;
            float d = orc_f16_to_f32_k256(ld16(blk));
            for (int ib = 0; ib < 8; ++ib) {
                float dl = d * (float)(iq4xs_ls(blk, ib) - 32);
                for (int j = 0; j < 16; ++j) {
                    uint8_t q = blk[8 + 16 * ib + j];
                    o[32 * ib + j] = dl * (float)orc_iq4nl_values[q & 15];
                    o[32 * ib + 16 + j] = dl * (float)orc_iq4nl_values[q >> 4];
                }
            }
        } else {
            const uint8_t *blk = w + 210 * b;
            float d = orc_f16_to_f32_k256(ld16(blk + 208));
            const int8_t *sc = (const int8_t *)(blk + 192);
            for (int e = 0; e < 256; ++e) {
                int h = e / 128, q = (e % 128) / 32, l = e % 32;
                int lo = (q & 1) ? blk[64 * h + 32 + l] : blk[64 * h + l];
                lo = (q >= 2) ? (lo >> 4) : (lo & 15);
                int hb = (blk[128 + 32 * h + l] >> (2 * q)) & 3;
                o[e] = d * (float)sc[e / 16] * (float)((lo | (hb << 4)) - 32);
            }
        }
    }
    return 0;
}
