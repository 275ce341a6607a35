// api.hip -- extern "C" entry points of include/qwen35_hip.h: argument
// validation, path dispatch and the ragged packer.  No arithmetic on the
// host: every result comes from a kernel in this library.
#include "../../include/qwen35_hip.h"
#include "qhip_device.hpp"
#include "qhip_internal.hpp"

#include <climits>
#include <cstdio>
#include <cstring>

namespace qhip {

static bool geom(int ttype, int& be, int& bb) {
  switch (ttype) {
    case TT_Q8_0: be = 32; bb = 34; return true;
    case TT_IQ4_NL: be = 32; bb = 18; return true;
    case TT_Q4_0: be = 32; bb = 18; return true;
    case TT_Q4_1: be = 32; bb = 20; return true;
    case TT_Q4_K: be = 256; bb = 144; return true;
    case TT_Q6_K: be = 256; bb = 210; return true;
    case TT_Q5_K: be = 256; bb = 176; return true;
    case TT_Q3_K: be = 256; bb = 110; return true;
    case TT_Q2_K: be = 256; bb = 84; return true;
    case TT_IQ4_XS: be = 256; bb = 136; return true;
    case TT_IQ3_XXS: be = 256; bb = 98; return true;
    case TT_IQ3_S: be = 256; bb = 110; return true;
    default: return false;
  }
}

static int act_elems(int ttype) {
  int be, bb;
  if (!geom(ttype, be, bb)) return 0;
  return be == 32 ? 32 : 256;
}

static long act_row_bytes(int ttype, int cols) {
  const int ab = act_elems(ttype);
  if (!ab || cols <= 0 || cols % ab) return -1;
  return ab == 32 ? (long)cols / 32 * 34 : (long)cols / 256 * 292;
}

static long weight_row_bytes(int ttype, int cols) {
  int be, bb;
  if (!geom(ttype, be, bb) || cols <= 0 || cols % be) return -1;
  if (act_row_bytes(ttype, cols) < 0) return -1;
  return (long)cols / be * bb;
}

static bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }

// Preconditions of the unit-decode kernels (see qhip_device.hpp): every load
// is a dword-aligned access inside the weight or activation buffer, which
// requires 4-byte aligned bases, whole 64-value units, and a total weight
// size that is a multiple of 4 (Q6_K pieces are read from the dword at or
// below their 2-byte aligned start).
static bool fast_ok(const GemvArgs& g) {
  if (!aligned4(g.w) || !aligned4(g.xq)) return false;
  if (g.cols % 64) return false;
  if (((long)g.rows * g.row_bytes) % 4) return false;
  return true;
}

static hipError_t make_args(const void* w, const void* xq, float* out, int rows, int cols,
                            int tokens, int ttype, GemvArgs& g) {
  if (!w || !xq || !out || rows < 0 || tokens < 0) return hipErrorInvalidValue;
  const long rb = weight_row_bytes(ttype, cols);
  const long ab = act_row_bytes(ttype, cols);
  if (rb < 0 || ab < 0) return hipErrorInvalidValue;
  if ((long)tokens > 65535L * 64) return hipErrorInvalidValue;
  g = GemvArgs{ttype, w, xq, out, rows, cols, tokens, rb, ab};
  return hipSuccess;
}

// Token count from which the MMQ tiles beat the weight-streaming GEMV, both
// at their defaults (the MMQ with the split-K workspace the Exec mirror
// passes).  Measured on MI355X: Q4_K [17408, 5120] (the weights-direct MMQ)
// GEMV 18.7 / MMQ 19.7 us at 4 tokens, 22.5 / 19.7 at 5; Q6_K [5120, 17408] (the few-token
// weights-direct MMQ on the GGUF rows) 27.2 / 31.5 at 4, 37.1 / 31.5 at 6; IQ4_NL [17408, 5120] 30.8 /
// 34.7 at 8, 46.4 / 34.7 at 12;
// Q8_0 [3584, 1024] 7.8 / 8.7 at 16; Q3_K / Q2_K [17408, 5120] 48.6 / 29.6
// and 38.6 / 26.8 us at 8 (Q2_K 23.3 / 26.5 at 4).
static int mmq_min_tokens(int ttype) {
  switch (ttype) {
    case TT_Q4_K: return 5;
    case TT_Q5_K: case TT_Q6_K: return 6;
    case TT_IQ4_XS: case TT_IQ3_XXS: case TT_IQ3_S: case TT_Q3_K: case TT_Q2_K: return 8;
    case TT_IQ4_NL: case TT_Q4_0: case TT_Q4_1: return 10;
    default: return 24;
  }
}

// Formats with an MMQ kernel: all of them.
static bool mmq_supported(int ttype) {
  return act32(ttype) || iq3(ttype) || ttype == TT_Q4_K || ttype == TT_Q6_K || ttype == TT_Q5_K ||
         ttype == TT_IQ4_XS || ttype == TT_Q3_K || ttype == TT_Q2_K;
}

// The Exec mirror multiplies Q6_K weights by many tokens from their plane
// image (built once per weight).  Measured on MI355X with the weights streamed
// from HBM, [5120, 17408]: 48.8 / 51.9 / 53.1 / 64.7 / 76.3 / 124.6 us at 64 /
// 96 / 128 / 192 / 256 / 512 tokens, against 49.0 / 77.8 / 78.7 / 160.9 /
// 231.3 / 293.2 for the GGUF-row MMQ (the previous, row-major Q6_K image:
// 54.0 / 59.6 / 61.2 / 82.0 / 106.9 / 205.9).  Up to 64 tokens the fragment
// image (46.9 us at 64).  Q4_K stays on its fragment image: its MMQ image's
// 3.9x larger weight bytes cost more than the scaling they save.
bool mmq_image_preferred(const GemvArgs& g) {
  return g.ttype == TT_Q6_K && g.tokens > 64 && mmq_image_bytes(g.ttype, g.rows, g.cols) > 0 && fast_ok(g);
}

// Batches of a large Q6_K or Q4_K weight: the Exec mirror multiplies them
// from the weight's fragment image (the GGUF bytes once more, permuted).
// Measured on MI355X with the weights streamed from HBM (rotated copies):
// Q6_K [5120, 17408] 19.6 / 20.0 / 21.0 / 26.4 / 36.4 us at 2 / 4 / 8 / 16 /
// 32 tokens from the image, against GEMV 18.2 / 25.3 / 33.5 / 49.0 us at 1 /
// 2 / 4 / 8 and the GGUF-row MMQ 33.0 / 33.4 / 33.4 / 38.0 / 43.8 us; Q4_K
// [17408, 5120] 13.0 / 13.4 / 14.2 / 17.5 / 22.6 / 35.2 / 145.9 us at 2 / 4 /
// 8 / 16 / 32 / 64 / 512 tokens, against GEMV 11.4 / 15.0 / 21.0 / 33.1 us at
// 1 / 2 / 4 / 8 and the GGUF-row MMQ 19.7 / 20.0 / 19.7 / 21.2 / 25.7 / 39.8 /
// 154.0 us.  The image from 2 tokens (at one the GEMV is ahead: 12.7 / 19.5
// us from the images); Q6_K up to its 64-token limit (two 32-token tiles side
// by side from 33: 46.8 / 46.9 us at 48 / 64 tokens against 49.4 / 49.1 from
// the plane image and about 50 from the GGUF-row MMQ), the plane image
// beyond.
//
// Q8_0 (the image MMQ from 6 tokens where K is one 1024-value super-chunk):
// measured on MI355X, [3584, 1024] GEMV 3.59 / 4.36 / 4.84 / 7.84 / 14.02 us
// at 4 / 6 / 8 / 16 / 32 tokens against 4.23 / 4.25 / 4.32 / 4.47 / 4.90
// from the image (the GGUF-row MMQ 9.4 us at 16); 64 / 512 / 1673 tokens
// 7.0 / 11.5 / 28.0 us against 9.7 / 12.6 / 30.0 on the GGUF rows.  With K
// = 3584 ([1024, 3584]: 16 workgroups walking four super-chunks) the image
// loses to the GEMV up to 24 tokens (13.3 against 16.9 us there), so wider
// Q8_0 rows keep the GGUF-row paths.
bool wd_image_preferred(const GemvArgs& g) {
  if (g.ttype == TT_Q8_0)
    return g.tokens >= 6 && g.cols <= 1024 && wd_image_bytes(g.ttype, g.rows, g.cols) > 0 && fast_ok(g);
  if (g.tokens < 2 || (long)g.rows * g.cols < (1L << 23) || !fast_ok(g)) return false;
  if (g.ttype == TT_Q6_K) return g.tokens <= 64 && wd_image_bytes(g.ttype, g.rows, g.cols) > 0;
  return g.ttype == TT_Q4_K && wd_image_bytes(g.ttype, g.rows, g.cols) > 0;
}

// `work` (nullable): the split-K workspace of the MMQ (mmq_work_bytes)
hipError_t dispatch_mul_mat(const GemvArgs& g, int path, void* work, long work_bytes, hipStream_t s) {
  if (g.rows == 0 || g.tokens == 0) return hipSuccess;
  const bool fast = fast_ok(g);
  switch (path) {
    case QHIP_PATH_GENERIC: return launch_gemv_generic(g, s);
    case QHIP_PATH_GEMV: return fast ? launch_gemv(g, 0, 0, 0, s) : launch_gemv_generic(g, s);
    case QHIP_PATH_MMQ:
      return fast && mmq_supported(g.ttype) ? launch_mmq(g, 0, 0, work, work_bytes, s) : (hipError_t)QHIP_DECLINE;
    case QHIP_PATH_AUTO:
      if (!fast) return launch_gemv_generic(g, s);
      if (mmq_supported(g.ttype) && g.tokens >= mmq_min_tokens(g.ttype)) return launch_mmq(g, 0, 0, work, work_bytes, s);
      return launch_gemv(g, 0, 0, 0, s);
    default: return hipErrorInvalidValue;
  }
}

// Workspace the MMQ of this product may split K into: the tile MMQ's and, for
// the formats with a weight image, the image MMQ's (the larger of the two);
// 0 when neither splits.
long mul_mat_work_bytes(const GemvArgs& g) {
  if (!fast_ok(g) || !mmq_supported(g.ttype)) return 0;
  long n = mmq_work_bytes(g);
  if (mmq_image_bytes(g.ttype, g.rows, g.cols) > 0) {
    const long m = mmq_image_work_bytes(g);
    if (m > n) n = m;
  }
  if (wd_image_bytes(g.ttype, g.rows, g.cols) > 0) {
    const long m = wd_image_work_bytes(g);
    if (m > n) n = m;
  }
  return n;
}

// ---- ragged packer: one launch quantizes every sequence into the packed buffer
// Grid: x = blocks of a token row, y = packed token.  The owning sequence of
// packed token p is found by binary search over the offset table.
__device__ __forceinline__ int find_seq(const int* __restrict__ off, int nseq, int p) {
  int lo = 0, hi = nseq;  // off[lo] <= p < off[hi]
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (off[mid] <= p) lo = mid; else hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(256) void k_quantize_ragged_q8_0(const float* const* __restrict__ src,
                                                              const int* __restrict__ off, int nseq,
                                                              uint8_t* __restrict__ out, long nblocks,
                                                              long cols, long out_stride) {
  const long b = ((long)blockIdx.x * 256 + threadIdx.x) >> 5;
  const int i = threadIdx.x & 31;
  const int p = blockIdx.y;
  const int sq = find_seq(off, nseq, p);
  const float* x = src[sq] + (long)(p - off[sq]) * cols;
  const bool ok = b < nblocks;
  const float v = ok ? x[32 * b + i] : 0.0f;
  uint32_t hb;
  const int q = quant_q8_0_lane(v, hb);
  if (ok) {
    uint8_t* ob = out + (long)p * out_stride + 34 * b;
    ob[2 + i] = (uint8_t)(int8_t)q;
    if (i == 0) {
      ob[0] = (uint8_t)hb;
      ob[1] = (uint8_t)(hb >> 8);
    }
  }
}

__global__ __launch_bounds__(256) void k_quantize_ragged_q8_K(const float* const* __restrict__ src,
                                                              const int* __restrict__ off, int nseq,
                                                              uint8_t* __restrict__ out, long nblocks,
                                                              long cols, long out_stride) {
  const long b = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  const int p = blockIdx.y;
  const int sq = find_seq(off, nseq, p);
  const float* x = src[sq] + (long)(p - off[sq]) * cols;
  const bool ok = b < nblocks;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = ok ? x[256 * b + 4 * l + i] : 0.0f;
  int gsum;
  float scale;
  const uint32_t packed = quant_q8_K_lane(v, gsum, scale);
  if (ok) {
    uint8_t* ob = out + (long)p * out_stride + 292 * b;
    *(uint32_t*)(ob + 4 + 4 * l) = packed;
    if ((l & 3) == 0) *(int16_t*)(ob + 260 + 2 * (l >> 2)) = (int16_t)gsum;
    if (l == 0) *(float*)ob = scale;
  }
}

}  // namespace qhip

using namespace qhip;

static hipStream_t S(void* s) { return (hipStream_t)s; }

// ---- probe ----------------------------------------------------------------------

static int g_arch = -2, g_cus = 0;
static char g_name[256] = "";

static void probe() {
  if (g_arch != -2) return;
  int dev = 0;
  hipDeviceProp_t p;
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess) {
    g_arch = -1;
    return;
  }
  int num = 0;
  const char* a = p.gcnArchName;
  if (a && !strncmp(a, "gfx", 3)) num = (int)strtol(a + 3, nullptr, 10);
  g_arch = num;
  g_cus = p.multiProcessorCount;
  snprintf(g_name, sizeof g_name, "%s (%s)", p.name, a ? a : "?");
}

extern "C" {

int qhip_init(int device) {
  hipError_t e = hipSetDevice(device);
  if (e != hipSuccess) return (int)e;
  g_arch = -2;
  probe();
  if (g_arch != 950) {
    fprintf(stderr, "qwen35_hip: device %d is %s, this library is built for gfx950 only\n",
            device, g_name);
    return (int)hipErrorInvalidDevice;
  }
  return (int)scratch_init_current_device();
}

int qhip_gpu_arch(void) { probe(); return g_arch; }
int qhip_gpu_cu_count(void) { probe(); return g_cus; }
const char* qhip_gpu_name(void) { probe(); return g_name; }

const char* qhip_error_string(int err) {
  if (err == QHIP_DECLINE) return "declined: this kernel path does not serve the request";
  return hipGetErrorString((hipError_t)err);
}

int qhip_quant_act_block_elems(int ttype) { return act_elems(ttype); }

int qhip_quant_geom(int ttype, int* block_elems, int* block_bytes) {
  int be, bb;
  if (!geom(ttype, be, bb)) return 0;
  if (block_elems) *block_elems = be;
  if (block_bytes) *block_bytes = bb;
  return 1;
}

long qhip_act_row_bytes(int ttype, int cols) { return act_row_bytes(ttype, cols); }
long qhip_weight_row_bytes(int ttype, int cols) { return weight_row_bytes(ttype, cols); }

int qhip_launch_quantize_q8_0(const float* d_x, void* d_out, int nblocks, void* stream) {
  if (nblocks < 0 || (nblocks > 0 && (!d_x || !d_out))) return (int)hipErrorInvalidValue;
  return (int)launch_quantize_q8_0(d_x, d_out, nblocks, 1, 0, 0, S(stream));
}

int qhip_launch_quantize_q8_K(const float* d_x, void* d_out, int nblocks, void* stream) {
  if (nblocks < 0 || (nblocks > 0 && (!d_x || !d_out))) return (int)hipErrorInvalidValue;
  if (!aligned4(d_out)) return (int)hipErrorInvalidValue;
  return (int)launch_quantize_q8_K(d_x, d_out, nblocks, 1, 0, 0, S(stream));
}

int qhip_launch_quantize_act(int ttype, const float* d_x, void* d_out, int cols, int tokens,
                             void* stream) {
  const long ab = act_row_bytes(ttype, cols);
  if (ab < 0 || tokens < 0 || tokens > 65535) return (int)hipErrorInvalidValue;
  if (tokens == 0) return 0;
  if (!d_x || !d_out) return (int)hipErrorInvalidValue;
  if (act_elems(ttype) == 32)
    return (int)launch_quantize_q8_0(d_x, d_out, cols / 32, tokens, cols, ab, S(stream));
  if (!aligned4(d_out)) return (int)hipErrorInvalidValue;
  return (int)launch_quantize_q8_K(d_x, d_out, cols / 256, tokens, cols, ab, S(stream));
}

int qhip_launch_dequantize(int ttype, const void* d_src, float* d_dst, int nblocks, void* stream) {
  int be, bb;
  if (!geom(ttype, be, bb) || nblocks < 0) return (int)hipErrorInvalidValue;
  if (nblocks == 0) return 0;
  if (!d_src || !d_dst) return (int)hipErrorInvalidValue;
  return (int)launch_dequant(ttype, d_src, d_dst, (long)nblocks * be, S(stream));
}

int qhip_launch_dequantize_row(int ttype, const void* d_src_row, float* d_dst, int cols, void* stream) {
  int be, bb;
  if (!geom(ttype, be, bb) || cols < 0 || cols % be) return (int)hipErrorInvalidValue;
  if (cols == 0) return 0;
  if (!d_src_row || !d_dst) return (int)hipErrorInvalidValue;
  return (int)launch_dequant(ttype, d_src_row, d_dst, cols, S(stream));
}

int qhip_launch_mul_mat(const void* d_w, const void* d_xq, float* d_out, int rows, int cols,
                        int tokens, int ttype, int path, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_w, d_xq, d_out, rows, cols, tokens, ttype, g);
  if (e != hipSuccess) return (int)e;
  return (int)dispatch_mul_mat(g, path, nullptr, 0, S(stream));
}

long qhip_mul_mat_work_bytes(int rows, int cols, int tokens, int ttype) {
  alignas(16) static const uint8_t dummy[16] = {};  // 16-byte aligned stand-ins: only the shape matters
  GemvArgs g;
  if (rows <= 0 || tokens <= 0 || make_args(dummy, dummy, (float*)dummy, rows, cols, tokens, ttype, g) != hipSuccess)
    return 0;
  return mul_mat_work_bytes(g);
}

int qhip_launch_mul_mat_work(const void* d_w, const void* d_xq, float* d_out, int rows, int cols, int tokens,
                             int ttype, int path, void* d_work, long work_bytes, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_w, d_xq, d_out, rows, cols, tokens, ttype, g);
  if (e != hipSuccess) return (int)e;
  if (work_bytes < 0 || (d_work && ((uintptr_t)d_work & 15u))) return (int)hipErrorInvalidValue;
  return (int)dispatch_mul_mat(g, path, d_work, d_work ? work_bytes : 0, S(stream));
}

int qhip_launch_mul_mat_vec(const void* d_w, const void* d_xq, float* d_out, int rows, int cols,
                            int tokens, int ttype, void* stream) {
  return qhip_launch_mul_mat(d_w, d_xq, d_out, rows, cols, tokens, ttype, QHIP_PATH_AUTO, stream);
}

int qhip_launch_mul_mat_vec_q8_0(const void* d_w, const void* d_xq, float* d_out, int rows,
                                 int cols, int tokens, void* stream) {
  return qhip_launch_mul_mat_vec(d_w, d_xq, d_out, rows, cols, tokens, QHIP_TT_Q8_0, stream);
}

int qhip_launch_quantize_mul_mat_vec(const void* d_w, const float* d_x, void* d_xq_out, float* d_out,
                                     int rows, int cols, int ttype, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_w, d_x, d_out, rows, cols, 1, ttype, g);
  if (e != hipSuccess) return (int)e;
  if (d_xq_out && !aligned4(d_xq_out)) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  // float4 activation reads: x 16-byte aligned
  if (!fast_ok(g) || ((uintptr_t)d_x & 15u) || !gemv_fused_fits(ttype, cols)) return QHIP_DECLINE;
  return (int)launch_gemv_fused(g, d_x, d_xq_out, 0, 0, 0, S(stream));
}

int qhip_launch_quantize_mul_mat_vec_tuned(const void* d_w, const float* d_x, void* d_xq_out, float* d_out, int rows,
                                           int cols, int ttype, int lanes_per_row, int rows_per_lane,
                                           int workgroup_threads, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_w, d_x, d_out, rows, cols, 1, ttype, g);
  if (e != hipSuccess) return (int)e;
  if (d_xq_out && !aligned4(d_xq_out)) return (int)hipErrorInvalidValue;
  const int wgs = workgroup_threads, nr = rows_per_lane;
  if (lanes_per_row < 0 || lanes_per_row > 64 || nr < 0 || nr > 4 || nr == 3 ||
      (wgs != 0 && wgs != 256 && wgs != 512 && wgs != 1024) || (wgs > 256 && nr > 2))
    return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!fast_ok(g) || ((uintptr_t)d_x & 15u) || !gemv_fused_fits(ttype, cols)) return QHIP_DECLINE;
  return (int)launch_gemv_fused(g, d_x, d_xq_out, lanes_per_row, nr, wgs, S(stream));
}

long qhip_quantize_mul_mat_vec_work_bytes(int rows, int cols) {
  if (rows < 0 || cols < 0) return 0;
  return gemv_splitk_work_bytes(rows, cols);
}

int qhip_launch_quantize_mul_mat_vec_split(const void* d_w, const float* d_x, void* d_xq_out, float* d_out,
                                           int rows, int cols, int ttype, int slice_values, int lanes_per_row,
                                           int rows_per_lane, void* d_work, long work_bytes, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_w, d_x, d_out, rows, cols, 1, ttype, g);
  if (e != hipSuccess) return (int)e;
  if (d_xq_out && !aligned4(d_xq_out)) return (int)hipErrorInvalidValue;
  if (slice_values < 0 || slice_values % 256 || lanes_per_row < 0 || lanes_per_row > 64 ||
      (lanes_per_row & (lanes_per_row - 1)) || (lanes_per_row > 0 && lanes_per_row < 4) || rows_per_lane < 0 ||
      rows_per_lane > 4 || rows_per_lane == 3)
    return (int)hipErrorInvalidValue;
  if (!d_work || ((uintptr_t)d_work & 15u) || work_bytes < gemv_splitk_work_bytes(rows, cols))
    return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!fast_ok(g) || ((uintptr_t)d_x & 15u) || cols % 256) return QHIP_DECLINE;
  if (slice_values && !gemv_fused_fits(ttype, slice_values)) return QHIP_DECLINE;
  return (int)launch_gemv_splitk(g, d_x, d_xq_out, lanes_per_row, rows_per_lane, slice_values, d_work, work_bytes,
                                 S(stream));
}

int qhip_launch_gemv_tuned(const void* d_w, const void* d_xq, float* d_out, int rows, int cols,
                           int tokens, int ttype, int lanes_per_row, int tokens_per_pass,
                           int rows_per_lane, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_w, d_xq, d_out, rows, cols, tokens, ttype, g);
  if (e != hipSuccess) return (int)e;
  const int n = tokens_per_pass, nr = rows_per_lane;
  const bool multiwave = lanes_per_row == 128 || lanes_per_row == 256;
  if (lanes_per_row < 0 || (lanes_per_row > 64 && !multiwave) || n < 0 || n > 8 || (n & (n - 1)))
    return (int)hipErrorInvalidValue;
  if (nr < 0 || nr > 4 || nr == 3) return (int)hipErrorInvalidValue;
  if (multiwave && (tokens != 1 || n > 1)) return (int)hipErrorInvalidValue;
  if (!fast_ok(g)) return QHIP_DECLINE;
  return (int)launch_gemv(g, lanes_per_row, n, nr, S(stream));
}

int qhip_launch_mmq_tuned(const void* d_w, const void* d_xq, float* d_out, int rows, int cols,
                          int tokens, int ttype, int tile_tokens, int tile_rows, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_w, d_xq, d_out, rows, cols, tokens, ttype, g);
  if (e != hipSuccess) return (int)e;
  const bool bt_ok = tile_tokens == 0 || tile_tokens == 64 || tile_tokens == 128 ||
                     (tile_tokens == 32 && (tile_rows == 128 || tile_rows == 64));
  const bool br_ok = tile_rows == 0 || tile_rows == 64 || tile_rows == 128;
  if (!bt_ok || !br_ok) return (int)hipErrorInvalidValue;
  if (!fast_ok(g) || !mmq_supported(ttype)) return QHIP_DECLINE;
  return (int)launch_mmq(g, tile_tokens, tile_rows, nullptr, 0, S(stream));
}

long qhip_mmq_image_bytes(int ttype, int rows, int cols) { return mmq_image_bytes(ttype, rows, cols); }

int qhip_launch_mmq_prepare(int ttype, const void* d_w, int rows, int cols, void* d_image, void* stream) {
  const long rb = weight_row_bytes(ttype, cols);
  if (rb < 0 || mmq_image_bytes(ttype, rows, cols) < 0) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!d_w || !d_image || ((uintptr_t)d_image & 15u)) return (int)hipErrorInvalidValue;
  return (int)launch_mmq_prepare(ttype, d_w, rb, rows, cols, d_image, S(stream));
}

int qhip_launch_mul_mat_image(const void* d_image, const void* d_xq, float* d_out, int rows, int cols,
                              int tokens, int ttype, int tile_tokens, int tile_rows, void* d_work,
                              long work_bytes, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_image, d_xq, d_out, rows, cols, tokens, ttype, g);
  if (e != hipSuccess) return (int)e;
  if (mmq_image_bytes(ttype, rows, cols) < 0) return (int)hipErrorInvalidValue;
  // Q6_K's plane-image MMQ has one shape: only the default
  const bool tile_ok = (tile_tokens == 0 && tile_rows == 0) ||
                       (ttype != TT_Q6_K && ((tile_tokens == 64 && tile_rows == 64) ||
                                             (tile_tokens == 64 && tile_rows == 128) ||
                                             (tile_tokens == 128 && tile_rows == 64)));
  if (!tile_ok || ((uintptr_t)d_image & 15u) || !aligned4(d_xq)) return (int)hipErrorInvalidValue;
  if (work_bytes < 0 || (d_work && ((uintptr_t)d_work & 15u))) return (int)hipErrorInvalidValue;
  return (int)launch_mmq_image(g, tile_tokens, tile_rows, d_work, d_work ? work_bytes : 0, S(stream));
}

long qhip_wd_image_bytes(int ttype, int rows, int cols) { return wd_image_bytes(ttype, rows, cols); }

int qhip_launch_wd_prepare(int ttype, const void* d_w, int rows, int cols, void* d_image, void* stream) {
  const long rb = weight_row_bytes(ttype, cols);
  if (rb < 0 || wd_image_bytes(ttype, rows, cols) < 0) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!d_w || !d_image || ((uintptr_t)d_image & 15u)) return (int)hipErrorInvalidValue;
  return (int)launch_wd_prepare(ttype, d_w, rb, rows, cols, d_image, S(stream));
}

int qhip_launch_mul_mat_wd_image(const void* d_image, const void* d_xq, float* d_out, int rows, int cols,
                                 int tokens, int ttype, void* d_work, long work_bytes, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_image, d_xq, d_out, rows, cols, tokens, ttype, g);
  if (e != hipSuccess) return (int)e;
  if (wd_image_bytes(ttype, rows, cols) < 0 || (ttype == TT_Q6_K && tokens > 64)) return (int)hipErrorInvalidValue;
  if (((uintptr_t)d_image & 15u) || !aligned4(d_xq)) return (int)hipErrorInvalidValue;
  if (work_bytes < 0 || (d_work && ((uintptr_t)d_work & 15u))) return (int)hipErrorInvalidValue;
  if (rows == 0 || tokens == 0) return 0;
  return (int)launch_mmq_wd_image(g, d_work, d_work ? work_bytes : 0, S(stream));
}

// whether a GEMV image exists for this format and width: the 32-value
// formats at the widths their team geometry covers, Q4_K / Q6_K at whole
// super-blocks
static bool gemv_image_ok(int ttype, int cols) {
  if (gemv_kimage_format(ttype)) return cols > 0 && cols % 256 == 0;
  return gemv_image_format(ttype) && gemv_image_width(cols);
}

long qhip_gemv_image_bytes(int ttype, int rows, int cols) {
  const long rb = weight_row_bytes(ttype, cols);
  if (rb < 0 || rows < 0 || !gemv_image_ok(ttype, cols)) return -1;
  return (long)rows * rb;
}

long qhip_gemv_image_act_bytes(int ttype, int cols, int tokens) {
  if (weight_row_bytes(ttype, cols) < 0 || !gemv_image_ok(ttype, cols) || tokens < 0) return -1;
  // Q4_K / Q6_K images read the reference Q8_K rows
  if (gemv_kimage_format(ttype)) return act_row_bytes(ttype, cols) * tokens;
  return gemv_image_act_bytes(cols, tokens);
}

int qhip_launch_gemv_prepare(int ttype, const void* d_w, int rows, int cols, void* d_image, void* stream) {
  const long rb = weight_row_bytes(ttype, cols);
  if (qhip_gemv_image_bytes(ttype, rows, cols) < 0) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!d_w || !d_image || !aligned4(d_w) || ((uintptr_t)d_image & 15u) || d_image == d_w)
    return (int)hipErrorInvalidValue;
  if (gemv_kimage_format(ttype)) return (int)launch_kimage_prepare(ttype, d_w, rb, rows, cols, d_image, S(stream));
  return (int)launch_gemv_image_prepare(d_w, rb, rows, cols, d_image, S(stream), ttype);
}

int qhip_launch_quantize_act_image(int ttype, const float* d_x, void* d_xa, int cols, int tokens, void* stream) {
  if (qhip_gemv_image_act_bytes(ttype, cols, tokens) < 0 || tokens > 65535) return (int)hipErrorInvalidValue;
  if (tokens == 0) return 0;
  if (!d_x || !d_xa || !aligned4(d_x) || ((uintptr_t)d_xa & 15u)) return (int)hipErrorInvalidValue;
  if (gemv_kimage_format(ttype)) return qhip_launch_quantize_act(ttype, d_x, d_xa, cols, tokens, stream);
  return (int)launch_quantize_act_image(ttype, d_x, d_xa, cols, tokens, cols, S(stream));
}

int qhip_launch_mul_mat_vec_image(const void* d_image, const void* d_xa, float* d_out, int rows, int cols,
                                  int ttype, int rows_per_lane, void* stream) {
  const long rb = weight_row_bytes(ttype, cols);
  if (qhip_gemv_image_bytes(ttype, rows, cols) < 0) return (int)hipErrorInvalidValue;
  if (rows_per_lane < 0 || rows_per_lane > 2) return (int)hipErrorInvalidValue;
  if (rows == 0) return 0;
  if (!d_image || !d_xa || !d_out || ((uintptr_t)d_image & 15u) || ((uintptr_t)d_xa & 15u))
    return (int)hipErrorInvalidValue;
  if (gemv_kimage_format(ttype)) {
    GemvArgs g{ttype, d_image, d_xa, d_out, rows, cols, 1, rb, act_row_bytes(ttype, cols)};
    g.kimg = true;
    return (int)launch_gemv(g, 0, 0, rows_per_lane, S(stream));
  }
  const GemvArgs g{ttype, d_image, d_xa, d_out, rows, cols, 1, rb, gemv_image_act_bytes(cols, 1)};
  return (int)launch_gemv_image(g, rows_per_lane, S(stream));
}

int qhip_launch_mul_mat_vec_tile(const void* d_w, const void* d_xq, float* d_out, int rows, int cols,
                                 int tokens, int ttype, void* stream) {
  return qhip_launch_mul_mat(d_w, d_xq, d_out, rows, cols, tokens, ttype, QHIP_PATH_MMQ, stream);
}

int qhip_ragged_offsets(const int* lengths, int nseq, int* offsets) {
  if (!lengths || !offsets || nseq < 0) return -1;
  long acc = 0;
  offsets[0] = 0;
  for (int i = 0; i < nseq; ++i) {
    if (lengths[i] < 0) return -1;
    acc += lengths[i];
    if (acc > INT_MAX) return -1;
    offsets[i + 1] = (int)acc;
  }
  return (int)acc;
}

int qhip_launch_quantize_ragged(int ttype, const float* const* d_src, const int* d_offsets,
                                int nseq, int total_tokens, int cols, void* d_xq_packed,
                                void* stream) {
  const long ab = act_row_bytes(ttype, cols);
  if (ab < 0 || nseq < 0 || total_tokens < 0 || total_tokens > 65535) return (int)hipErrorInvalidValue;
  if (total_tokens == 0) return 0;
  if (nseq == 0 || !d_src || !d_offsets || !d_xq_packed) return (int)hipErrorInvalidValue;
  // Q8_0: the wide form for large batches when the output allows (rows of
  // any 4-byte alignment)
  if (act_elems(ttype) == 32 && quantize_wide_preferred((long)(cols / 32) * total_tokens) &&
      ((uintptr_t)d_xq_packed & 1u) == 0 && (ab & 1) == 0)
    return (int)launch_quantize_wide(true, nullptr, d_src, d_offsets, nseq, d_xq_packed, cols / 32, total_tokens,
                                     cols, ab, S(stream));
  if (act_elems(ttype) == 32) {
    const long nb = cols / 32;
    dim3 grid((unsigned)((nb * 32 + 255) / 256), (unsigned)total_tokens);
    hipLaunchKernelGGL(k_quantize_ragged_q8_0, grid, dim3(256), 0, S(stream), d_src, d_offsets,
                       nseq, (uint8_t*)d_xq_packed, nb, (long)cols, ab);
  } else {
    if (!aligned4(d_xq_packed)) return (int)hipErrorInvalidValue;
    const long nb = cols / 256;
    dim3 grid((unsigned)((nb + 3) / 4), (unsigned)total_tokens);
    hipLaunchKernelGGL(k_quantize_ragged_q8_K, grid, dim3(256), 0, S(stream), d_src, d_offsets,
                       nseq, (uint8_t*)d_xq_packed, nb, (long)cols, ab);
  }
  return (int)hipGetLastError();
}

int qhip_launch_mul_mat_ragged(const void* d_w, const void* d_xq_packed, float* d_out, int rows,
                               int cols, const int* d_offsets, int nseq, int total_tokens,
                               int ttype, void* stream) {
  if (nseq < 0 || (nseq > 0 && !d_offsets)) return (int)hipErrorInvalidValue;
  GemvArgs g;
  hipError_t e = make_args(d_w, d_xq_packed, d_out, rows, cols, total_tokens, ttype, g);
  if (e != hipSuccess) return (int)e;
  return (int)dispatch_mul_mat(g, QHIP_PATH_AUTO, nullptr, 0, S(stream));
}

int qhip_launch_block_ints(const void* d_w, const void* d_xq, int32_t* d_ints, int rows, int cols,
                           int tokens, int ttype, void* stream) {
  GemvArgs g;
  hipError_t e = make_args(d_w, d_xq, reinterpret_cast<float*>(d_ints), rows, cols, tokens, ttype, g);
  if (e != hipSuccess) return (int)e;
  if (!fast_ok(g)) return (int)hipErrorInvalidValue;
  return (int)launch_block_ints(g, d_ints, S(stream));
}

}  // extern "C"
