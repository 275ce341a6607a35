// scratch.hip -- the split-K quantize + GEMV for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc).  Same kernels and results as
// qhip_launch_quantize_mul_mat_vec_split; the workspace (row-tile counters and
// per-slice partial sums) is a file-scope device array instead of a caller
// buffer.
//
// The array's name is a host-side stand-in in host code, not a device
// address: its address on each device comes from hipGetSymbolAddress, taken
// once per device with that device current (qhip_init, or the entry point's
// first call on a device), and only that pointer is ever passed to a kernel.
// Every call on one device shares that device's array: calls that overlap on
// one GPU (two streams, or two host threads) race on it.
#include "../../include/qwen35_hip.h"
#include "qhip_internal.hpp"

#include <mutex>

namespace qhip {

// 4 MiB per device: 32 KiB of row-tile counters + partial sums for
// rows * ceil(cols / 256) <= 1,040,384 (e.g. [5120, 17408] needs 348,160).
constexpr long kScratchBytes = 4L << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// Resolve the current device's copy of the array and clear its counters
// (a fill kernel on `s`, so the clear is ordered before any launch on `s`;
// under capture it becomes a graph node, harmless on replay because the
// counters are zero again after every launch).
static hipError_t scratch_ptr(hipStream_t s, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    e = launch_fill_zero(p, kSkCountBytes, s);
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

// Called by qhip_init with the device current: set-up outside any capture,
// finished before qhip_init returns.
hipError_t scratch_init_current_device() {
  void* p = nullptr;
  hipError_t e = scratch_ptr(nullptr, &p);
  if (e != hipSuccess) return e;
  return hipStreamSynchronize(nullptr);
}

}  // namespace qhip

using namespace qhip;

extern "C" int qhip_launch_quantize_mul_mat_vec_split_noalloc(const void* d_w, const float* d_x, void* d_xq_out,
                                                              float* d_out, int rows, int cols, int ttype,
                                                              int slice_values, int lanes_per_row,
                                                              int rows_per_lane, void* stream) {
  if (rows < 0 || cols < 0) return (int)hipErrorInvalidValue;
  // beyond the array: rejected before anything is launched
  if (gemv_splitk_work_bytes(rows, cols) > kScratchBytes) return (int)hipErrorInvalidValue;
  void* ws = nullptr;
  const hipError_t e = scratch_ptr((hipStream_t)stream, &ws);
  if (e != hipSuccess) return (int)e;
  return qhip_launch_quantize_mul_mat_vec_split(d_w, d_x, d_xq_out, d_out, rows, cols, ttype, slice_values,
                                                lanes_per_row, rows_per_lane, ws, kScratchBytes, stream);
}
