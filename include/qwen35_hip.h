/*
 * qwen35_hip.h -- C ABI of the MI355X (gfx950) quantized matvec / MMQ backend.
 *
 * This is the only surface a host engine sees.  It mirrors the reference's
 * device-kernel ABI (src/kernels/cuda/api.h) and its backend vtable slots for
 * the quantized-matvec path (src/backend.zig:110-178), so that a
 * backend_hip.zig can sit beside src/backend_cpu.zig: plain C types, device
 * pointers as `void *`, the stream as `void *` (a hipStream_t; NULL = the
 * default stream), no HIP or torch types in any signature.
 *
 * Conventions (as the reference, src/kernels/cuda/api.h:1-13):
 *   - launchers return the numeric hipError_t as int, 0 = success;
 *   - QHIP_DECLINE (-1) means "this path does not serve the request, use
 *     another one" (src/kernels/cuda/mmq.cu:2242-2245) -- never a silent CPU
 *     fallback; nothing in this library runs arithmetic on the host;
 *   - invalid type ids, shapes that are not a multiple of the block size, NULL
 *     buffers and out-of-range counts return hipErrorInvalidValue (1) before
 *     anything is launched (src/kernels/cuda/mmvq.cu:781-785 pattern).
 *
 * Type ids are the GGUF TensorType numbers (src/gguf.zig TensorType,
 * src/kernels/cuda/api.h:52-75).  Supported: Q8_0, Q4_K, Q6_K, IQ4_NL (the
 * benchmark formats), Q5_K, Q3_K, Q2_K, IQ4_XS, Q4_0, Q4_1, IQ3_XXS, IQ3_S.
 *
 * Layouts (all little-endian, GGUF block formats, src/gguf.zig:168-207):
 *   weight rows   rows x (cols / block_elems) blocks, rows contiguous
 *   Q8_0 act      34 B per 32 values: f16 d, int8 qs[32]
 *   Q8_K act      292 B per 256 values: f32 d, int8 qs[256], int16 bsums[16]
 *   output        float out[t * rows + r] = W[r] . x_t
 * Fast paths need 4-byte aligned weight and activation pointers, a weight
 * byte size that is a multiple of 4, and cols a multiple of 64; other inputs
 * take the byte-granular generic kernel.

 */
#ifndef QWEN35_HIP_H
#define QWEN35_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QHIP_TT_Q8_0 8
#define QHIP_TT_Q4_K 12
#define QHIP_TT_Q6_K 14
#define QHIP_TT_IQ4_NL 20
#define QHIP_TT_Q2_K 10
#define QHIP_TT_Q3_K 11
#define QHIP_TT_Q5_K 13
#define QHIP_TT_IQ4_XS 23
#define QHIP_TT_Q4_0 2
#define QHIP_TT_Q4_1 3
#define QHIP_TT_IQ3_XXS 18
#define QHIP_TT_IQ3_S 21

#define QHIP_DECLINE (-1)

/* Kernel path selection for qhip_launch_mul_mat. */
#define QHIP_PATH_AUTO 0    /* GEMV for small token counts, MMQ above the crossover */
#define QHIP_PATH_GEMV 1    /* weight-streaming GEMV, tokens share each weight load */
#define QHIP_PATH_MMQ 2     /* int8 MFMA tiles; declines (QHIP_DECLINE) if unsupported */
#define QHIP_PATH_GENERIC 3 /* byte-granular reference kernel, any alignment */

/* ---- device probe ---------------------------------------------------------
 * Replaces q35_gpu_cc / q35_gpu_sm_count / q35_gpu_name
 * (src/kernels/cuda/api.h:35-37) and the device check in CudaBackend.init
 * (src/backend_cuda.zig:1601-1625).  qhip_init makes `device` current for
 * the calling thread and fails with a HIP error if it is not a gfx950 GPU. */
int qhip_init(int device);
int qhip_gpu_arch(void);          /* e.g. 950 for gfx950; -1 without a device */
int qhip_gpu_cu_count(void);      /* compute units; 0 without a device */
const char *qhip_gpu_name(void);  /* marketing name, "" without a device */
const char *qhip_error_string(int err);

/* ---- geometry (pure host code) --------------------------------------------
 * q35_quant_act_block_elems / q35_quant_geom (src/kernels/cuda/api.h:444-449). */
int qhip_quant_act_block_elems(int ttype); /* 32 (Q8_0 act), 256 (Q8_K act), 0 unknown */
int qhip_quant_geom(int ttype, int *block_elems, int *block_bytes); /* 1 ok, 0 unknown */
/* Bytes of one quantized activation row / one packed weight row; -1 if invalid. */
long qhip_act_row_bytes(int ttype, int cols);
long qhip_weight_row_bytes(int ttype, int cols);

/* ---- activation quantization ----------------------------------------------
 * q35_launch_quantize_q8_0 / q35_launch_quantize_q8_K
 * (src/kernels/cuda/api.h:77-84), bit-exact with the CPU quantize_q8_0 /
 * quantize_q8_K (src/kernels/x86/kernels32.c:1064-1087,
 * kernels256.c:865-896).  `nblocks` counts 32- resp. 256-value blocks. */
int qhip_launch_quantize_q8_0(const float *d_x, void *d_out, int nblocks, void *stream);
int qhip_launch_quantize_q8_K(const float *d_x, void *d_out, int nblocks, void *stream);
/* `tokens` rows of `cols` floats -> the activation family of `ttype`
 * (backend_cpu.zig:42-50 actFamily), one quantized row per token. */
int qhip_launch_quantize_act(int ttype, const float *d_x, void *d_out, int cols, int tokens,
                             void *stream);

/* ---- dequantization ---------------------------------------------------------
 * q35_launch_dequantize (src/kernels/cuda/api.h:95-96): `nblocks` NATIVE blocks
 * (32 values for Q8_0 / IQ4_NL, 256 for Q4_K / Q6_K) of packed bytes to f32.
 * q35_launch_dequantize_row (api.h:101-102): one row of `cols` values.
 * Bit-exact with src/quant_dequant.zig (the CPU dequantRowInto,
 * src/backend_cpu.zig:661-679). */
int qhip_launch_dequantize(int ttype, const void *d_src, float *d_dst, int nblocks, void *stream);
int qhip_launch_dequantize_row(int ttype, const void *d_src_row, float *d_dst, int cols, void *stream);

/* ---- matvec -----------------------------------------------------------------
 * q35_launch_mul_mat_vec (src/kernels/cuda/api.h:104-112):
 *   out[t*rows + r] = W[r] . xq[t] for t < tokens.
 * d_xq holds `tokens` rows quantized with the weight's activation family.
 * These stateless launchers read the GGUF rows in every call.  The faster
 * weight-image kernels need an image built once per weight and are reached
 * through the Exec mirror (qhip_backend_*, which builds and keeps them) or
 * the explicit image entry points below.  Measured on MI355X: config 5 Q6_K
 * [5120, 17408] at 512 tokens 293.5 us here against 124.9 us from the plane
 * image; the config-3 IQ4_NL head [248320, 2560] at one token 71.2 us against
 * 61.6 us from the GEMV image. */
int qhip_launch_mul_mat_vec(const void *d_w, const void *d_xq, float *d_out, int rows, int cols,
                            int tokens, int ttype, void *stream);
/* q35_launch_mul_mat_vec_q8_0 (src/kernels/cuda/api.h:116-117). */
int qhip_launch_mul_mat_vec_q8_0(const void *d_w, const void *d_xq, float *d_out, int rows,
                                 int cols, int tokens, void *stream);
/* Same contract with an explicit kernel path (QHIP_PATH_*); replaces the
 * reference's env switches (QWEN35_CUDA_MMQ, src/kernels/cuda/mmvq.cu:553-586)
 * with an argument. */
int qhip_launch_mul_mat(const void *d_w, const void *d_xq, float *d_out, int rows, int cols,
                        int tokens, int ttype, int path, void *stream);
/* The same with a workspace the MMQ may split K into.  The launches above
 * never split K (each output tile is one workgroup's sum over all of K).
 * With few output tiles (a few dozen tokens) one workgroup per tile leaves
 * most of the GPU idle; given d_work of qhip_mul_mat_work_bytes(rows, cols,
 * tokens, ttype) bytes (16-byte aligned, its first 32 KiB zero before the
 * first launch -- hipMemset once at allocation -- and zero again after every
 * launch), the default MMQ cuts K into slices, and the last workgroup of each
 * tile adds the slices' partial tiles in slice order: results are the same on
 * every run (no float atomics).  With a smaller or NULL d_work, K is not
 * split.  Launches that share a d_work must not overlap (one stream).
 * qhip_mul_mat_work_bytes is 0 when no split would be made.  No reference
 * counterpart (the reference's MMQ never splits K, src/kernels/cuda/mmq.cu:
 * 1197-1202). */
long qhip_mul_mat_work_bytes(int rows, int cols, int tokens, int ttype);
int qhip_launch_mul_mat_work(const void *d_w, const void *d_xq, float *d_out, int rows, int cols,
                             int tokens, int ttype, int path, void *d_work, long work_bytes, void *stream);

/* Quantize-and-multiply for one token in ONE launch: d_x is the f32
 * activation (16-byte aligned); every workgroup quantizes it with the
 * reference quantizer of the weight's activation family (bit-exact with
 * qhip_launch_quantize_act) into LDS and runs the GEMV on it.  d_xq_out
 * (nullable) receives the quantized activation in the reference layout.
 * Replaces the reference's quantize launch + matvec launch pair
 * (src/backend_cuda.zig matvec path: q35_launch_quantize_q8_0/_q8_K then
 * q35_launch_mul_mat_vec, src/kernels/cuda/api.h:79-112); no reference kernel
 * fuses them.  Returns QHIP_DECLINE when the fast-path preconditions do not
 * hold or cols is too wide for the LDS image (about 57000 values). */
int qhip_launch_quantize_mul_mat_vec(const void *d_w, const float *d_x, void *d_xq_out, float *d_out,
                                     int rows, int cols, int ttype, void *stream);

/* The one-launch quantize + GEMV with an explicit shape: `lanes_per_row`
 * (1..64) lanes share `rows_per_lane` (1, 2 or 4) rows; `workgroup_threads`
 * 256, 512 or 1024 (512 / 1024 with at most two rows per lane) quantize the
 * activation once per workgroup; 0 picks for any of them.  Replaces nothing
 * in the reference (its launch shapes are env knobs,
 * src/kernels/cuda/mmvq.cu:685-772).  Declines as
 * qhip_launch_quantize_mul_mat_vec. */
int qhip_launch_quantize_mul_mat_vec_tuned(const void *d_w, const float *d_x, void *d_xq_out, float *d_out,
                                           int rows, int cols, int ttype, int lanes_per_row, int rows_per_lane,
                                           int workgroup_threads, void *stream);

/* The same product for long rows, split over K: each workgroup quantizes and
 * multiplies one slice of `slice_values` values (a multiple of 256; 0 picks)
 * of a tile of rows, writes its partial sums into d_work, and the last
 * workgroup of each row tile to finish adds the partials in slice order
 * (deterministic).  `lanes_per_row` (4, 8, 16, 32 or 64) and `rows_per_lane`
 * (1, 2 or 4) set the shape; 0 picks.  d_work holds
 * qhip_quantize_mul_mat_vec_work_bytes(rows, cols) bytes; its first 32 KiB
 * must be zero before the first launch (hipMemset once at allocation) and
 * are zero again after every launch.  Launches that share a d_work must not
 * overlap (one stream).  Replaces the same reference pair as above for the
 * FFN down projection's long rows, where quantizing the whole activation in
 * every workgroup does not pay; no reference kernel splits K.  Returns
 * QHIP_DECLINE when the fast-path preconditions do not hold. */
long qhip_quantize_mul_mat_vec_work_bytes(int rows, int cols);
int qhip_launch_quantize_mul_mat_vec_split(const void *d_w, const float *d_x, void *d_xq_out, float *d_out,
                                           int rows, int cols, int ttype, int slice_values,
                                           int lanes_per_row, int rows_per_lane, void *d_work,
                                           long work_bytes, void *stream);

/* The split-K quantize + GEMV above WITHOUT a workspace argument, for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  Same kernels, arguments and results as
 * qhip_launch_quantize_mul_mat_vec_split; the workspace is a 4 MiB array the
 * library holds on each device it runs on until the process ends, so
 * rows * ceil(cols / 256) may be at most 1,040,384 (larger shapes return
 * hipErrorInvalidValue before anything is launched).  It calls no
 * hipMalloc / hipFree.  Every call on one device shares that device's array:
 * calls that overlap on one GPU (two streams or two host threads) race and
 * must be serialized by the caller.  qhip_init sets the array up for its
 * device; on a device qhip_init was not called for, the first call does. */
int qhip_launch_quantize_mul_mat_vec_split_noalloc(const void *d_w, const float *d_x, void *d_xq_out,
                                                   float *d_out, int rows, int cols, int ttype,
                                                   int slice_values, int lanes_per_row, int rows_per_lane,
                                                   void *stream);

/* The GEMV with explicit launch shape: `lanes_per_row` (1..64, or 128 / 256
 * = two / four whole waves, one token only) lanes share `rows_per_lane` (1, 2
 * or 4) weight rows, walking their 64-value units in turn, and fold their
 * partial sums; `tokens_per_pass` in {1,2,4,8} tokens share each weight load;
 * 0 picks the default for any of them.  Replaces the reference's launch-shape env knobs
 * (QWEN35_CUDA_SPLIT / _COOP_WARPS / _RPB, src/kernels/cuda/mmvq.cu:685-772)
 * with arguments.  Returns QHIP_DECLINE when the fast-path preconditions do
 * not hold. */
int qhip_launch_gemv_tuned(const void *d_w, const void *d_xq, float *d_out, int rows, int cols,
                           int tokens, int ttype, int lanes_per_row, int tokens_per_pass,
                           int rows_per_lane, void *stream);

/* ---- batched prefill on int8 MFMA tiles (MMQ) -----------------------------------
 * q35_launch_mul_mat_vec_tile (src/kernels/cuda/mmq.cu:2232-2336): the same
 * product as qhip_launch_mul_mat_vec for a batch of tokens, on 32x32 int8 MFMA
 * tiles.  Returns QHIP_DECLINE when the fast-path preconditions above do not
 * hold (the caller then uses qhip_launch_mul_mat_vec, as mmvq.cu:789-800 does).
 * Unlike the reference it serves every type here (Q8_0 included) and any
 * token count. */
int qhip_launch_mul_mat_vec_tile(const void *d_w, const void *d_xq, float *d_out, int rows,
                                 int cols, int tokens, int ttype, void *stream);
/* The MMQ with an explicit workgroup tile: `tile_tokens` x `tile_rows`
 * outputs, each 64 or 128, or 32 x 128 / 32 x 64 (0 picks).  Replaces the reference's compile-time
 * tile constants (mmq.cu, 128 rows x 8 tokens per CTA) with arguments.
 * Returns QHIP_DECLINE when the fast-path preconditions do not hold. */
int qhip_launch_mmq_tuned(const void *d_w, const void *d_xq, float *d_out, int rows, int cols,
                          int tokens, int ttype, int tile_tokens, int tile_rows, void *stream);

/* MMQ weight image (no reference counterpart; the reference's CUDA MMQ decodes
 * the GGUF blocks in every launch, mmq.cu:499-659).  For Q4_K and Q6_K the
 * integer sub-block scales are folded into the quantized values once,
 * p = sc*q (Q4_K) or sc*(q6-32) (Q6_K), split exactly into two int8 planes
 * p = 2^S*hi + lo, so the MMQ accumulates a whole super-block on the matrix
 * core without per-group integer scaling.  Q4_K: row-major planes, 560 bytes
 * per 256 weights.  Q6_K: the planes in MFMA fragment order per 32-row group
 * (16,512 bytes per 32 rows and 256 values, about 516 per 256 weights).
 *   qhip_mmq_image_bytes   image size, -1 for other types or cols % 256 != 0
 *   qhip_launch_mmq_prepare  build it from GGUF bytes (d_image 16-byte aligned)
 *   qhip_launch_mul_mat_image  the product from the image: same contract and
 *     results as qhip_launch_mul_mat_vec_tile; Q4_K tile 64x64 / 64x128 /
 *     128x64 tokens x rows, 0 x 0 = default; Q6_K only 0 x 0 (its kernel has
 *     one shape: a persistent grid over 128-row tiles of 64 or 128 tokens);
 *     d_work (nullable) as for qhip_launch_mul_mat_work
 *     (qhip_mul_mat_work_bytes covers the image launch too); without a
 *     large enough d_work no Q6_K tile is cut over K (the launch runs
 *     unsplit, with the same results) */
long qhip_mmq_image_bytes(int ttype, int rows, int cols);
int qhip_launch_mmq_prepare(int ttype, const void *d_w, int rows, int cols, void *d_image, void *stream);
int qhip_launch_mul_mat_image(const void *d_image, const void *d_xq, float *d_out, int rows, int cols,
                              int tokens, int ttype, int tile_tokens, int tile_rows, void *d_work,
                              long work_bytes, void *stream);

/* Fragment images of Q6_K, Q4_K and Q8_0 weights (no reference counterpart; the
 * reference's CUDA MMQ decodes the GGUF blocks in every launch,
 * mmq.cu:499-659, and declines Q8_0 to its GEMV, mmq.cu:2250-2264).  The GGUF
 * bytes permuted -- the same bytes per row and 256 values -- so that the
 * weights-direct MMQ loads each matrix-core fragment as
 * one aligned, contiguous 1 KB per wave instruction (a GGUF row's blocks
 * otherwise give a wave instruction 32 rows' pieces, most of them misaligned
 * for Q6_K's 210-byte blocks).  Rows in groups of 32, the last padded with
 * zero rows; group r, super-block b is one tile at (r * cols/256 + b) * tile:
 *   Q6_K, 6720-byte tiles: [0, 6144) lane L = i + 32k (row i, value half k)
 *     holds 24 dwords, dwords 4c..4c+3 at 1024c + 16L; dwords 6j..6j+5
 *     (j = 2h + m) are the 8 bytes of ql at 64h + 16m + 8k, of ql at
 *     64h + 32 + 16m + 8k and of qh at 128 + 32h + 16m + 8k; [6144, 6656) row
 *     i's 16 scales at 16i; [6656, 6720) row i's f16 d at 2i.
 *   Q4_K, 4608-byte tiles: [0, 4096) lane L holds qs bytes 32c + 16k .. +15
 *     of row i at 1024c + 16L (c < 4); [4096, 4608) row i's 16-byte header
 *     (d, dmin, scales) at 16i.
 *   Q8_0, per group r (nb = cols/32 blocks) at r * nb * 1088: nb 1024-byte
 *     quant tiles (block b's at 1024b: lane L holds values 16k .. 16k+15 of
 *     row i at 16L), then nb runs of the 32 rows' f16 d (block b's at
 *     1024nb + 64b: row 8q + 4h + j at 2 (16h + 4q + j), the order of the
 *     rows in a lane's MFMA result elements).
 *   qhip_wd_image_bytes    image size, -1 unless ttype is Q6_K / Q4_K / Q8_0 and cols % 256 == 0
 *   qhip_launch_wd_prepare build it from GGUF bytes (d_image 16-byte aligned)
 *   qhip_launch_mul_mat_wd_image  d_out [tokens, rows] from the image (Q6_K
 *     1..64 tokens, Q4_K and Q8_0 any count; activations as for
 *     qhip_launch_mul_mat); d_work (nullable) as for qhip_launch_mul_mat_work,
 *     qhip_mul_mat_work_bytes covers it.  Q6_K / Q4_K: the same integers as
 *     the MMQ on the GGUF rows (QHIP_PATH_MMQ), and the same bits where the
 *     launches cut K alike; Q8_0: the same block integers, scaled as
 *     (da sumi) dw per block and added in four K quarters (within 1e-6
 *     relative of the GGUF-row MMQ), d_work unused */
long qhip_wd_image_bytes(int ttype, int rows, int cols);
int qhip_launch_wd_prepare(int ttype, const void *d_w, int rows, int cols, void *d_image, void *stream);
int qhip_launch_mul_mat_wd_image(const void *d_image, const void *d_xq, float *d_out, int rows, int cols,
                                 int tokens, int ttype, void *d_work, long work_bytes, void *stream);

/* GEMV weight image (no reference counterpart; the reference's CUDA GEMV reads
 * the GGUF blocks as they are, mmvq.cu).  For the 32-value formats (IQ4_NL,
 * Q4_0: 18-byte blocks; Q8_0: 34-byte blocks), whose blocks leave every
 * 16-byte piece of a row misaligned: the same bytes per row (36 / 68 per 64
 * values), reordered so that each 16-byte load of the GEMV is aligned and the
 * lanes of a team read one contiguous span -- the 16-byte quant pieces of
 * each block (one for the 4-bit formats, two for Q8_0) in the order the team
 * walks the row, then the f16 scales, each lane's adjacent.  The order depends on
 * the row width (the team width and pass count the library takes for it;
 * at width 5120 Q8_0 40 lanes and two passes, IQ4_NL 16 lanes and five);
 * widths 1024, 1280, 2048, 2560, 3072, 3840, 4096, 5120, 6144 and 8192
 * have one.  The activation of the image GEMV is quantized
 * into the matching split layout (the same Q8_0 values and scales as
 * qhip_launch_quantize_act; scales stored as f32): 72 bytes per 64 values.
 * For Q4_K and Q6_K (any cols % 256 == 0): the same bytes per row, each
 * 64-value unit's 16-byte pieces (Q4_K two quant pieces, Q6_K ql, ql, qh)
 * grouped by piece over chunks of 64 units, so that lanes on consecutive
 * units read one contiguous span per load; then the Q4_K super-block headers
 * (16 bytes each), or the Q6_K units' four scales (4 bytes each) and the f16
 * d of each super-block.  Its activation is the reference Q8_K row
 * (qhip_launch_quantize_act_image = qhip_launch_quantize_act), and the image
 * GEMV gives the same bits as qhip_launch_mul_mat_vec on the GGUF rows with
 * the same rows per lane -- except the Q6_K image's default launch from 4096
 * rows at widths of 64a + b units with a = 1 (b <= 32), 3 or 4, whose
 * balanced teams sum a row's units in another order (within 1e-6 relative
 * L2 of the GGUF-row launch; config 5's [5120, 17408] 15.4 us against 18.4).
 *   qhip_gemv_image_bytes      image size (rows x GGUF row bytes); -1 for
 *                              other types or widths
 *   qhip_gemv_image_act_bytes  bytes of `tokens` activation rows, or -1
 *   qhip_launch_gemv_prepare   build it from GGUF bytes (d_w 4-byte aligned,
 *                              d_image 16-byte aligned, not d_w)
 *   qhip_launch_quantize_act_image  f32 x[tokens][cols] -> split activation
 *                              (d_xa 16-byte aligned)
 *   qhip_launch_mul_mat_vec_image   out[r] = W[r] . x for one token from the
 *     image and the split activation: the integers of the GGUF-layout GEMV,
 *     floats within its tolerance.  rows_per_lane 1 or 2 (0 = the library's
 *     choice). */
long qhip_gemv_image_bytes(int ttype, int rows, int cols);
long qhip_gemv_image_act_bytes(int ttype, int cols, int tokens);
int qhip_launch_gemv_prepare(int ttype, const void *d_w, int rows, int cols, void *d_image, void *stream);
int qhip_launch_quantize_act_image(int ttype, const float *d_x, void *d_xa, int cols, int tokens, void *stream);
int qhip_launch_mul_mat_vec_image(const void *d_image, const void *d_xa, float *d_out, int rows, int cols,
                                  int ttype, int rows_per_lane, void *stream);

/* ---- ragged prefill (no reference counterpart: the reference prefills one
 * sequence per chunk, src/engine.zig:1371) -------------------------------------
 * Sequence i owns packed tokens [offsets[i], offsets[i+1]); offsets has
 * nseq+1 entries, offsets[0] = 0, offsets[nseq] = total_tokens.
 *
 * Packer: quantizes each sequence's f32 rows (d_src[i] -> lengths from the
 * offset table) into the packed activation buffer, in one launch.  d_src is a
 * DEVICE array of nseq device pointers; d_offsets is a device array. */
int qhip_launch_quantize_ragged(int ttype, const float *const *d_src, const int *d_offsets,
                                int nseq, int total_tokens, int cols, void *d_xq_packed,
                                void *stream);
/* Host helper: offsets[0..nseq] = prefix sums of lengths; returns the total,
 * or -1 for a negative length or overflow. */
int qhip_ragged_offsets(const int *lengths, int nseq, int *offsets);
/* One launch over all sequences: out[p*rows + r] = W[r] . xq[p] for every
 * packed token p (GEMV or MMQ by the total token count).  Every packed token
 * row is an independent product, so MMQ token tiles may span sequences. */
int qhip_launch_mul_mat_ragged(const void *d_w, const void *d_xq_packed, float *d_out, int rows,
                               int cols, const int *d_offsets, int nseq, int total_tokens,
                               int ttype, void *stream);

/* ---- parity export -----------------------------------------------------------
 * Exact per-block integers through the same unit decode as the GEMV kernels:
 * ints[(t*rows + r)*nints + i], nints = cols/block_elems, except the formats
 * with mins: Q4_K, Q5_K, Q2_K store (isum, summs) per super-block (nints =
 * 2*cols/256), Q4_1 (sumi, sumy) per block (nints = 2*cols/32); IQ4_XS,
 * IQ3_XXS and IQ3_S one integer per 32-value sub-block before its scale
 * (nints = cols/32).  The integers of
 * src/kernels/x86/kernels32.c:447-464 / :342-361 / :297-340 and
 * kernels256.c:474-498 / :720-738. */
int qhip_launch_block_ints(const void *d_w, const void *d_xq, int32_t *d_ints, int rows, int cols,
                           int tokens, int ttype, void *stream);

/* ---- backend (mirror of the Exec vtable's quantized-matvec slots) -----------
 * src/backend.zig:110-178.  A backend owns device copies of weights
 * (loadLinear, backend.zig:115-119; upload as in backend_cuda.zig:3458),
 * activation scratch (allocScratch/allocScratchK/freeScratch, :133-139) and
 * Buf regions (allocBuf, :141-146).  All matvec inputs/outputs are device
 * pointers (Buf), so consecutive ops never cross PCIe. */
typedef struct qhip_backend qhip_backend;

/* LinearW.quant (backend.zig:47-50, gguf.zig QuantRow:312-365): a resident,
 * packed 2-D weight. */
typedef struct qhip_linear {
  const void *dev;  /* device bytes, GGUF block layout */
  int ttype;
  int rows;
  int cols;
  long row_bytes;
} qhip_linear;

qhip_backend *qhip_backend_create(int device, int *err);
void qhip_backend_destroy(qhip_backend *be);
/* name()/describe() (backend.zig:493-498) */
const char *qhip_backend_name(const qhip_backend *be);
/* Upload `rows` packed rows from host memory.  Weights are placed back to back
 * in a device arena, so two consecutive loads of the same shape are adjacent
 * (the condition matvecPair fuses on, backend_cuda.zig:3743-3794). */
int qhip_backend_load_linear(qhip_backend *be, int ttype, int rows, int cols,
                             const void *host_data, qhip_linear *out);
/* Adopt weights already resident on this device (no copy, not freed).  Call
 * qhip_backend_free_linear before the caller releases or reuses that memory:
 * it drops what the backend derived from the bytes (the MMQ and GEMV
 * images). */
int qhip_backend_wrap_linear(qhip_backend *be, int ttype, int rows, int cols, const void *d_data,
                             qhip_linear *out);
void qhip_backend_free_linear(qhip_backend *be, qhip_linear *w);
/* Build what this weight's products use beyond its GGUF bytes now, at load
 * time, instead of inside the first matvec: the GEMV image of an IQ4_NL /
 * Q4_0 / Q8_0 weight large enough for the decode matvec to read it, or of a
 * Q6_K weight whose decode matvec quantizes separately (widths above 4096, or
 * more than 32768 rows)
 * (qhip_launch_gemv_prepare, the GGUF bytes once more; built in load order,
 * so adjacent weights get adjacent images and matvecPair stays one launch),
 * the fragment image of a Q6_K or Q4_K weight with rows * cols >= 2^23
 * (qhip_launch_wd_prepare, the GGUF bytes once more; matvec_batch_k reads it
 * from 2 tokens, Q6_K up to 64) or of a Q8_0 weight with cols <= 1024 (from
 * 6 tokens) and the MMQ image of a Q6_K weight
 * (qhip_launch_mmq_prepare, 2.5x the GGUF bytes; from 65 tokens).
 * 0 = built or nothing to build; QHIP_DECLINE = not all built (images off, or
 * past the memory budget): the products then read the GGUF bytes.
 * No reference counterpart (its CUDA kernels decode the GGUF blocks in every
 * launch). */
int qhip_backend_prepare_linear(qhip_backend *be, const qhip_linear *w);
/* MMQ images (the fragment images and the Q6_K MMQ image) on (default) or
 * off; off, matvec_batch_k never builds or reads one. */
int qhip_backend_set_mmq_images(qhip_backend *be, int on);
/* GEMV images on (default) or off; off, matvec never builds or reads one. */
int qhip_backend_set_gemv_images(qhip_backend *be, int on);
/* Cap on the device bytes this backend places (uploaded weights, MMQ images,
 * scratch, workspaces, allocBuf regions); 0 = no cap (the default).
 * QWEN35_CUDA_MAX_DEV_MIB of src/backend_cuda.zig:1754-1760 as an argument:
 * a load or buffer past it fails with hipErrorOutOfMemory and a message; an
 * MMQ image past it is simply not built.  mem_placed: bytes counted so far. */
int qhip_backend_set_mem_budget(qhip_backend *be, size_t bytes);
size_t qhip_backend_mem_placed(const qhip_backend *be);
int qhip_backend_alloc_scratch(qhip_backend *be, int max_cols);
int qhip_backend_alloc_scratch_k(qhip_backend *be, int max_cols, int k);
void qhip_backend_free_scratch(qhip_backend *be);
/* allocBuf: `len` floats of device memory owned by the backend until
 * free_scratch / destroy. */
int qhip_backend_alloc_buf(qhip_backend *be, size_t len, float **d_out);
/* matvec (backend.zig:153-158): d_out[rows] = W . d_x[cols] (f32 in, f32 out). */
int qhip_backend_matvec(qhip_backend *be, float *d_out, const qhip_linear *w, const float *d_x);
/* matvecPair (backend.zig:159-176): out[0..r) = A.x, out[r..2r) = B.x; one
 * quantization and one launch when A and B are adjacent and alike, else two. */
int qhip_backend_matvec_pair(qhip_backend *be, float *d_out, const qhip_linear *a,
                             const qhip_linear *b, const float *d_x);
/* matvecBatchK (backend.zig:177-178): out[j*rows + r] = W[r] . x_j, j < k. */
int qhip_backend_matvec_batch_k(qhip_backend *be, float *d_out, const qhip_linear *w,
                                const float *d_xK, int k);
/* dequantRow (backend.zig:148-151): d_dst[cols] = f32 values of weight row `row`
 * (the embedding lookup). */
int qhip_backend_dequant_row(qhip_backend *be, float *d_dst, const qhip_linear *w, int row);
/* Stream for subsequent calls (NULL = default stream) and a host wait.
 * Changing the stream forgets the memoized activation (below) and, unless
 * the old stream is being captured, waits for the old stream's work: the
 * backend's activation scratch and split-K workspace are single buffers, so
 * launches on two streams must not overlap. */
int qhip_backend_set_stream(qhip_backend *be, void *stream);
int qhip_backend_sync(qhip_backend *be);

/* Activation-quantization memo (src/backend_cuda.zig:3425-3448 actQValid /
 * actQMark, used by the matvec slot at :3914-3944).  When on, a matvec whose
 * x pointer, width, token count and activation family (Q8_0 or Q8_K) match
 * the last quantization reuses the quantized rows in the scratch instead of
 * quantizing again (q/k/v of one hidden state, Q4_K and Q6_K weights of one
 * x, the halves of a non-adjacent matvecPair).  Off by default.  The caller
 * must call qhip_backend_act_invalidate after anything writes into a buffer
 * a matvec may read again (the reference clears at the same points,
 * backend_cuda.zig:6250-6254: rmsnorm, l2norm, add_resid, copy_range,
 * copy_from_host, swiglu, mul_silu, dequant_row, load_linear, const_buf).
 * set_act_memo also clears it. */
int qhip_backend_set_act_memo(qhip_backend *be, int on);
void qhip_backend_act_invalidate(qhip_backend *be);
/* Memo hits and misses since create (the reference's QWEN35_QSTAT counters,
 * backend_cuda.zig:3933-3937); either pointer may be NULL. */
int qhip_backend_act_stats(const qhip_backend *be, unsigned long long *hits,
                           unsigned long long *misses);
/* Decode-step boundary (src/backend.zig:470-491 stepBegin/stepEnd).  A device
 * backend may ignore the hint; this one clears the activation memo at
 * step_begin (as backend_cuda.zig:7049-7053 does) and captures nothing.  An
 * engine can wrap a step in its own HIP graph: under capture the backend
 * allocates nothing -- it builds no MMQ image (the tile MMQ runs instead) and
 * grows no workspace (an MMQ that would need more runs unsplit) -- but the
 * activation scratch must already be large enough, so run the step once
 * eagerly (or call alloc_scratch_k and prepare_linear) before capturing.
 * Once a capture has been seen, a scratch or workspace that a later eager
 * call outgrows is kept, not freed, until free_scratch / destroy, so a graph
 * captured earlier never names freed memory. */
void qhip_backend_step_begin(qhip_backend *be, unsigned pos);
void qhip_backend_step_end(qhip_backend *be);

/* ---- introspection and profiling of the backend -------------------------------
 * describe() (src/backend.zig:494-495): a one-line account of what is in use --
 * device, CU count, the bytes of weights, images, scratch and the budget, and
 * which images, the memo and profiling are on.  The string belongs to the
 * backend and stays valid until the next describe call or destroy. */
const char *qhip_backend_describe(qhip_backend *be);
/* Device timing of the slots (the Exec profiling slots reportProfile /
 * profReport, src/backend.zig:500-514; the reference's per-type device table
 * and event-timed slots, src/backend_cuda.zig:6647 reportStats, :6195
 * slotEnter).  With profiling on, every matvec, matvec_pair, matvec_batch_k
 * and dequant_row call records a HIP event pair on the backend's stream
 * around its launches; the pairs are read back lazily (at most 512
 * outstanding: the oldest half is waited for when the queue fills), so the
 * slots still return without a host wait.  Times are summed per (slot,
 * type, rows, cols, tokens) with the calls' algorithmic bytes (packed
 * weights + 4 cols tokens + 4 rows tokens; dequant_row: one row + 4 cols) and
 * int8 ops (2 rows cols tokens).  Calls made while the stream is being
 * captured into a graph are not timed, only counted (prof_untimed).  Off by
 * default; the binding turns it on under $QWEN35_PROF as the reference does. */
#define QHIP_SLOT_MATVEC 0
#define QHIP_SLOT_MATVEC_PAIR 1
#define QHIP_SLOT_MATVEC_BATCH_K 2
#define QHIP_SLOT_DEQUANT_ROW 3
typedef struct qhip_prof_entry {
  int slot;         /* QHIP_SLOT_* */
  int ttype;
  int rows;         /* matvec_pair: the two weights' rows together */
  int cols;
  int tokens;
  long long calls;
  double device_us; /* summed over the calls */
  double bytes;     /* summed algorithmic bytes */
  double ops;       /* summed int8 ops */
} qhip_prof_entry;
int qhip_backend_set_profiling(qhip_backend *be, int on);
/* Waits for every recorded pair, then writes up to max_entries rows, largest
 * device time first; returns the number of rows the table has. */
int qhip_backend_prof_entries(qhip_backend *be, qhip_prof_entry *out, int max_entries);
/* The same table as text (a header line, then one `HIP-PROF` line per row
 * with calls, total and average device us, GB/s, the fraction of the 8 TB/s
 * HBM peak and TOP/s), NUL-terminated in buf[0..len); returns the length of
 * the whole text (snprintf semantics), -1 on a bad argument. */
long qhip_backend_prof_report(qhip_backend *be, char *buf, long len);
long long qhip_backend_prof_untimed(const qhip_backend *be);
void qhip_backend_prof_reset(qhip_backend *be);

#ifdef __cplusplus
}
#endif
#endif /* QWEN35_HIP_H */
