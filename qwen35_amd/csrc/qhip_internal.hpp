// qhip_internal.hpp -- launch functions shared between the kernel files and
// the C-ABI layer (api.hip).  Not part of the public interface.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qhip {

struct GemvArgs {
  int ttype;
  const void* w;     // packed weight rows, GGUF block layout
  const void* xq;    // quantized activations, reference layout, `tokens` rows
  float* out;        // [tokens][rows]
  int rows, cols, tokens;
  long row_bytes;    // bytes of one weight row
  long act_bytes;    // bytes of one quantized activation row
  bool kimg = false;  // w is a Q4_K / Q6_K GEMV image (one token)
};

hipError_t launch_quantize_q8_0(const float* x, void* out, long nblocks, int tokens, long x_stride,
                                long out_stride, hipStream_t s);
hipError_t launch_quantize_q8_K(const float* x, void* out, long nblocks, int tokens, long x_stride,
                                long out_stride, hipStream_t s);
// The wide quantizers (16-byte aligned f32 rows, x_stride a multiple of 4;
// Q8_0 output 2-byte aligned, Q8_K 4-byte): q8_0 selects the format.  With
// src (ragged) token t of the launch is packed token t: row src[i] + (t -
// off[i]) x_stride of its sequence i.
hipError_t launch_quantize_wide(bool q8_0, const float* x, const float* const* src, const int* off, int nseq,
                                void* out, long nblocks, int tokens, long x_stride, long out_stride,
                                hipStream_t s);
// whether the wide forms beat the one-block-per-lane-group ones at this many
// blocks (measured rule)
bool quantize_wide_preferred(long blocks);

// Waves a GEMV launch aims for (8 per CU on 256 CUs) when choosing lanes per row.
constexpr int kGemvTargetWaves = 2048;
int gemv_pick_team(int rows, int cols, int target_waves);
int gemv_pick_nt(int tokens);
// team: lanes per row group (0 = pick), nt: tokens per pass (0 = pick),
// nr: rows per lane (1, 2 or 4; 0 = 1)
hipError_t launch_gemv(const GemvArgs& g, int team, int nt, int nr, hipStream_t s);
hipError_t launch_gemv_generic(const GemvArgs& g, hipStream_t s);
hipError_t launch_block_ints(const GemvArgs& g, int* ints, hipStream_t s);
// Quantize + GEMV in one launch for one token: x is f32, the activation is
// quantized inside every workgroup (bit-exact with the quantizers) into LDS;
// xq_out (nullable) receives it in the reference layout.
constexpr long kFusedMaxLds = 64 * 1024;
bool gemv_fused_fits(int ttype, int cols);
// whether the fused launch beats quantize + GEMV for this shape (measured rule)
bool gemv_fused_preferred(const GemvArgs& g);
// team / nr / wgs (workgroup threads: 256, or 512 / 1024 with nr <= 2) 0 = pick
hipError_t launch_gemv_fused(const GemvArgs& g, const float* x, void* xq_out, int team, int nr, int wgs,
                             hipStream_t s);
// Split-K quantize + GEMV for one token on long rows: slices of `slice`
// values (a multiple of 256) per workgroup, partial sums in `work`
// (gemv_splitk_work_bytes; its first kSkCountBytes must be zero before the
// first launch and are zero again after each).  0 picks team / nr / slice.
constexpr long kSkMaxTiles = 8192;
constexpr long kSkCountBytes = 4 * kSkMaxTiles;
long gemv_splitk_work_bytes(int rows, int cols);
// zero `bytes` (a multiple of 4) with a fill kernel (no memset node in graphs)
hipError_t launch_fill_zero(void* p, long bytes, hipStream_t s);
bool gemv_splitk_preferred(const GemvArgs& g);
hipError_t launch_gemv_splitk(const GemvArgs& g, const float* x, void* xq_out, int team, int nr, int slice,
                              void* work, long work_bytes, hipStream_t s);
// resolve (and clear) the no-allocation entry point's device array on the
// current device; qhip_init calls it
hipError_t scratch_init_current_device();
// GGUF blocks -> f32 (nvals = whole blocks' values)
hipError_t launch_dequant(int ttype, const void* src, float* dst, long nvals, hipStream_t s);
// MMQ tile: bt tokens x br rows per workgroup, each 64 or 128 (0 = pick).
// With the default tile, small grids split K when `work` holds
// mmq_work_bytes(g) bytes (its first kSkCountBytes zero, as for the split-K
// GEMV); otherwise, and with an explicit tile, K is not split.
hipError_t launch_mmq(const GemvArgs& g, int bt, int br, void* work, long work_bytes, hipStream_t s);
long mmq_work_bytes(const GemvArgs& g);
// MMQ weight image of a K-quant weight (sub-scales folded into two int8 planes)
long mmq_image_bytes(int ttype, int rows, int cols);
hipError_t launch_mmq_prepare(int ttype, const void* w, long row_bytes, int rows, int cols, void* img,
                              hipStream_t s);
// g.w = the image; bt x br tile (0 = default; splits K as launch_mmq); Q6_K
// (the plane image) has one shape and ignores bt, br
hipError_t launch_mmq_image(const GemvArgs& g, int bt, int br, void* work, long work_bytes, hipStream_t s);
// Q6_K plane image and its MMQ (mmq.hip); the workspace: bg_work_bytes (0:
// none needed), its first kSkCountBytes zero; nwg > 0 overrides the grid
long bg_image_bytes_q6k(int rows, int cols);
hipError_t launch_bg_prepare_q6k(const void* w, long row_bytes, int rows, int cols, void* img, hipStream_t s);
long bg_work_bytes(const GemvArgs& g, int nwg);
hipError_t launch_mmq_bg_q6k(const GemvArgs& g, void* work, long work_bytes, hipStream_t s, int nwg);
// Q6_K fragment image (the GGUF bytes permuted for the few-token MMQ)
long wd_image_bytes(int ttype, int rows, int cols);
hipError_t launch_wd_prepare(int ttype, const void* w, long row_bytes, int rows, int cols, void* img,
                             hipStream_t s);
hipError_t launch_mmq_wd_image(const GemvArgs& g, void* work, long work_bytes, hipStream_t s);
long mmq_image_work_bytes(const GemvArgs& g);
// the split-K workspace launch_mmq_wd_image takes (fragment image; 0 = none)
long wd_image_work_bytes(const GemvArgs& g);
// GEMV weight image of the 32-value 4-bit formats (gemv_image.hip): the same
// bytes per row, quant bytes 16-byte aligned in unit order, scales apart
bool gemv_image_format(int ttype);
bool gemv_image_width(int cols);  // a team width and pass count exist for this row width
// the split activation's layout for this format and width (16 T + P; -1
// none): formats of one layout share a quantized activation
int gemv_image_layout(int ttype, int cols);
long gemv_image_act_bytes(int cols, int tokens);
hipError_t launch_gemv_image_prepare(const void* w, long row_bytes, int rows, int cols, void* img, hipStream_t s,
                                     int ttype);
hipError_t launch_quantize_act_image(int ttype, const float* x, void* out, int cols, int tokens, long x_stride,
                                     hipStream_t s);
// g.w = the image, g.xq = one token's split activation; nr rows per team (1,
// 2; 0 = pick)
hipError_t launch_gemv_image(const GemvArgs& g, int nr, hipStream_t s);
// whether quantize + image GEMV beats the GGUF-layout launches (measured rule)
bool gemv_image_preferred(const GemvArgs& g);
// K-quant GEMV image (Q4_K, Q6_K; KImg in qhip_device.hpp): the same bytes
// per row, read by launch_gemv / launch_gemv_fused / launch_gemv_splitk when
// g.kimg, with the reference Q8_K activation
bool gemv_kimage_format(int ttype);
hipError_t launch_kimage_prepare(int ttype, const void* w, long row_bytes, int rows, int cols, void* img,
                                 hipStream_t s);
// whether the Exec mirror's batch-1 matvec reads a K-quant weight's image
bool gemv_kimage_preferred(const GemvArgs& g);

}  // namespace qhip
