/*
 * oracle.h -- CPU restatement of the reference's quantized matvec path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code.  It exists so that tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py can check the HIP kernels against the
 * reference's arithmetic, and time that arithmetic on the host.
 *
 * What it restates (paths relative to the reference repository):
 *   f16 <-> f32            src/kernels/x86/kernels32.c:45-98, kernels256.c:51-78
 *   quantize_q8_0          src/kernels/x86/kernels32.c:1064-1087
 *   quantize_q8_K          src/kernels/x86/kernels256.c:865-896
 *   Q8_0 x Q8_0            src/kernels/x86/kernels32.c:447-464, kernels512.c:53-81
 *   IQ4_NL x Q8_0          src/kernels/x86/kernels32.c:342-361 (+ iq_tables.zig:429-432)
 *   Q4_0 / Q4_1 x Q8_0     src/kernels/x86/kernels32.c:297-340
 *   IQ3_XXS / IQ3_S x Q8_K src/kernels/x86/iq_kernels.c:612-643, :1728-1772
 *                          (grids: src/iq_tables.zig:323-425, ksigns :42-61)
 *   Q4_K x Q8_K            src/kernels/x86/kernels256.c:105-125, :179-186, :474-498
 *   Q6_K x Q8_K            src/kernels/x86/kernels256.c:200-212, :720-738
 *   matvec / batch driver  src/backend_cpu.zig:167-289, :328-446; src/pool.zig:300-336, :468-550
 *   dequant (fixtures)     src/quant_dequant.zig:54-77, :78-103, :222-251, :347-360,
 *                          :362-415, :417-445, :1388-1402
 *
 * Float results follow the scalar / AVX-512-VNNI tier order (one sequential
 * per-block fold).  The reference's AVX2 tier folds Q4_K/Q6_K with 8-lane
 * FMA; integers are identical on every tier, floats are compared with a
 * tolerance.
 */
#ifndef QWEN35_ORACLE_H
#define QWEN35_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* gguf TensorType ids (reference src/gguf.zig TensorType, src/kernels/cuda/api.h:52-75) */
#define ORC_TT_Q8_0   8
#define ORC_TT_Q4_K  12
#define ORC_TT_Q6_K  14
#define ORC_TT_IQ4_NL 20
#define ORC_TT_Q2_K  10
#define ORC_TT_Q3_K  11
#define ORC_TT_Q5_K  13
#define ORC_TT_IQ4_XS 23
#define ORC_TT_Q4_0   2
#define ORC_TT_Q4_1   3
#define ORC_TT_IQ3_XXS 18
#define ORC_TT_IQ3_S  21

float    orc_f16_to_f32(uint16_t h);        /* kernels32.c:45-66 (+0 for -0)  */
float    orc_f16_to_f32_k256(uint16_t h);   /* kernels256.c:51-78 (keeps -0) */
uint16_t orc_f32_to_f16(float x);           /* kernels32.c:67-98, RNE, NaN->inf */

void orc_quantize_q8_0(int n, const float *x, uint8_t *out);
void orc_quantize_q8_K(int n, const float *x, uint8_t *out);

/* Exact per-block integers. */
int32_t orc_blk_q8_0(const uint8_t *w, const uint8_t *a);
int32_t orc_blk_iq4_nl(const uint8_t *w, const uint8_t *a);
void    orc_blk_q4_k(const uint8_t *w, const uint8_t *a, int32_t *isum, int32_t *summs);
int32_t orc_blk_q6_k(const uint8_t *w, const uint8_t *a);
void    orc_blk_q5_k(const uint8_t *w, const uint8_t *a, int32_t *isum, int32_t *summs);
void    orc_blk_q2_k(const uint8_t *w, const uint8_t *a, int32_t *isum, int32_t *summs);
int32_t orc_blk_q3_k(const uint8_t *w, const uint8_t *a);
int32_t orc_blk_iq4_xs(const uint8_t *w, const uint8_t *a, int ib);
int32_t orc_blk_q4_0(const uint8_t *w, const uint8_t *a);
void    orc_blk_q4_1(const uint8_t *w, const uint8_t *a, int32_t *sumi, int32_t *sumy);
/* IQ3 32-value sub-block ib of a super-block: the signed grid values times q8,
 * before the sub-block scale 2*ls+1 */
int32_t orc_blk_iq3_xxs(const uint8_t *w, const uint8_t *a, int ib);
int32_t orc_blk_iq3_s(const uint8_t *w, const uint8_t *a, int ib);
/* grid entry i (u32, byte j = value j) and the sign mask of 7-bit index i */
uint32_t orc_iq3xxs_grid(int i);
uint32_t orc_iq3s_grid(int i);
uint8_t  orc_ksigns(int i);

/* Geometry: returns 1 and fills the outputs for a supported type, else 0. */
int orc_geom(int ttype, int *block_elems, int *block_bytes);
/* 32 (Q8_0 activation) or 256 (Q8_K activation); 0 for an unknown type. */
int orc_act_block_elems(int ttype);
/* Bytes of one quantized activation row of `cols` values; -1 on bad input. */
long orc_act_bytes(int ttype, int cols);
/* Bytes of one packed weight row; -1 on bad input. */
long orc_row_bytes(int ttype, int cols);

/* One weight row against one quantized activation row (n = cols). */
float orc_dot(int ttype, int n, const void *w, const void *a);

/* Per-block integers of one row.  Q8_0 / IQ4_NL / Q4_0 / Q6_K write n/block ints;
 * Q4_K writes 2 per super-block: isum then summs; Q4_1 2 per block: sumi then
 * sumy (the activation's block sum).  Returns ints written, or -1. */
int orc_block_nints(int ttype);
int orc_row_block_ints(int ttype, int n, const void *w, const void *a, int32_t *out);

/* Quantize one f32 row with the type's activation family. 0 on success. */
int orc_quantize_act(int ttype, int cols, const float *x, uint8_t *out);

/* out[t*rows + r] = W[r] . x_t for k tokens (x is [k, cols] f32).
 * Quantizes each token once, then row-parallel dots over `nthreads` threads
 * with the reference pool's chunk rule.  Returns 0 on success. */
int orc_matvec_batch(int ttype, int rows, int cols, int k, const void *w,
                     const float *x, float *out, int nthreads);

/* Same driver over caller-supplied C functions with the reference's own
 * signatures: dot = float(int n, const void*, const void*),
 * quant = void(int n, const float*, uint8_t*).  Used to time the compiled
 * reference kernels with the same threading as the restatement. */
typedef float (*orc_dot_fn)(int n, const void *w, const void *a);
typedef void (*orc_quant_fn)(int n, const float *x, uint8_t *out);
int orc_matvec_batch_fn(orc_dot_fn dot, orc_quant_fn quant, int ttype, int rows,
                        int cols, int k, const void *w, const float *x, float *out,
                        uint8_t *act_scratch, int nthreads);

/* Dot phase only (activations already quantized, [k, act_bytes]). */
int orc_matvec_q_fn(orc_dot_fn dot, int ttype, int rows, int cols, int k,
                    const void *w, const uint8_t *act, float *out, int nthreads);

/* Dequantize one packed row into cols floats (fixture semantics). */
int orc_dequant_row(int ttype, int cols, const void *w, float *out);

/* Function pointers of the restated dots/quantizers, for orc_matvec_batch_fn. */
orc_dot_fn   orc_dot_fn_for(int ttype);
orc_quant_fn orc_quant_fn_for(int ttype);

/* oracle_simd.c: the host-ISA tier of the row dot (IQ4_NL / Q4_K / Q6_K AVX2,
 * Q8_0 AVX-512 VNNI or AVX2; other types and hosts without AVX2: the scalar
 * restatement), the tier's name, and the Q8_0 AVX2 form on its own. */
orc_dot_fn   orc_simd_dot_fn_for(int ttype);
const char  *orc_simd_tier(int ttype);
orc_dot_fn   orc_simd_dot_q8_0_avx2(void);

#ifdef __cplusplus
}
#endif
#endif
