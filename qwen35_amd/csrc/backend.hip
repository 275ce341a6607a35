// backend.hip -- the host side of the Exec vtable's quantized-matvec slots
// (reference src/backend.zig:110-178), the part a backend_hip.zig would
// forward to.  Behavioural spec: the reference device backend
// (src/backend_cuda.zig:3458-4400): weights are uploaded once at load time and
// stay resident; activations are quantized on the device into backend-owned
// scratch; matvecPair runs as one launch when the two weights are adjacent and
// alike (:3743-3794); a failed launch is reported, never replaced by a CPU
// computation (:26-31).
#include "../../include/qwen35_hip.h"
#include "qhip_internal.hpp"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <utility>
#include <vector>

namespace qhip {
hipError_t dispatch_mul_mat(const GemvArgs& g, int path, void* work, long work_bytes, hipStream_t s);
long mul_mat_work_bytes(const GemvArgs& g);
bool mmq_image_preferred(const GemvArgs& g);
bool wd_image_preferred(const GemvArgs& g);
}

using namespace qhip;

struct qhip_backend {
  int device = 0;
  hipStream_t stream = nullptr;
  // Weight arena: large device chunks, bump-allocated with 256-byte alignment,
  // so consecutive loads are contiguous on the device.
  struct Chunk { uint8_t* base; size_t size, used; };
  std::vector<Chunk> arena;
  std::vector<std::pair<void*, size_t>> bufs;  // allocBuf regions (freed by free_scratch)
  uint8_t* act = nullptr;        // quantized-activation scratch
  size_t act_cap = 0;
  // split-K partials and tile counters of the GEMV and MMQ launches
  // (counters zero between launches)
  uint8_t* skwork = nullptr;
  size_t skwork_cap = 0;
  // Once a launch of this backend has been captured into a graph, a scratch
  // or workspace buffer that has to grow is not freed: the graph still names
  // it and may be replayed.  Such buffers are kept here (and still count
  // against the budget) until free_scratch or destroy.
  bool graph_seen = false;
  std::vector<std::pair<void*, size_t>> retired;
  // MMQ images of Q6_K weights: the plane image of the prefill MMQ
  // (qhip_launch_mmq_prepare, kind kImgMmq) and the fragment image of the
  // few-token MMQ (qhip_launch_wd_prepare, kind kImgFrag), built by
  // prepare_linear or by the first product that reads them outside a graph
  // capture, kept until free_linear / destroy.  Keyed by the whole linear
  // (device bytes, type, rows, cols) and the kind: a different weight wrapped
  // at a reused address never meets a stale image.
  struct ImageKey {
    const void* dev;
    int ttype, rows, cols, kind;
    bool operator<(const ImageKey& o) const {
      if (dev != o.dev) return dev < o.dev;
      if (ttype != o.ttype) return ttype < o.ttype;
      if (rows != o.rows) return rows < o.rows;
      if (cols != o.cols) return cols < o.cols;
      return kind < o.kind;
    }
  };
  struct Image {
    void* p;
    size_t bytes;
  };
  std::map<ImageKey, Image> images;
  bool images_on = true;
  // GEMV images of the 32-value 4-bit formats (gemv_image.hip), keyed by the
  // device address of the first GGUF row they mirror.  Their bytes come from
  // a bump arena of their own, so images built in load order are adjacent
  // exactly when their weights are, and an adjacent matvecPair stays one
  // launch.  free_linear drops the entries over the weight's rows; the arena
  // memory is returned at destroy, as the weights' is.
  struct GImage {
    uint8_t* img;
    int ttype, rows, cols;
    long row_bytes;
  };
  std::map<const uint8_t*, GImage> gimages;
  struct Chunk2 { uint8_t* base; size_t size, used; };
  std::vector<Chunk2> img_arena;
  bool gemv_images_on = true;
  // Device-memory budget (QWEN35_CUDA_MAX_DEV_MIB, backend_cuda.zig:1754-1760,
  // as an argument): bytes this backend places on the device -- uploaded
  // weights, MMQ images, scratch, workspaces, allocBuf regions.  0 = no cap.
  // A load past the budget fails; an image past it is not built (the prefill
  // then runs the tile MMQ on the GGUF bytes).
  size_t budget = 0;
  size_t placed = 0;  // bytes counted against the budget
  // What `act` holds (backend_cuda.zig:3425-3448 actQValid/actQMark): the
  // source pointer, width, token count and activation family of the last
  // quantization, so a second matvec of the same x skips its quantize.
  // Off unless enabled; cleared by step_begin, act_invalidate, set_stream and
  // a scratch reallocation.
  bool memo_on = false;
  const float* memo_src = nullptr;
  int memo_cols = 0, memo_k = 0, memo_fam = -1;
  unsigned long long memo_hits = 0, memo_misses = 0;
  // Device timing of the slots (the Exec profiling slots, backend.zig:500-514;
  // the reference's per-type device table, backend_cuda.zig:6647): an event
  // pair on the backend's stream around each slot call, read back lazily, and
  // summed per (slot, type, rows, cols, tokens).  Calls under a graph
  // capture are counted as untimed (an event there would become a graph
  // node).
  struct ProfKey {
    int slot, ttype, rows, cols, tokens;
    bool operator<(const ProfKey& o) const {
      if (slot != o.slot) return slot < o.slot;
      if (ttype != o.ttype) return ttype < o.ttype;
      if (rows != o.rows) return rows < o.rows;
      if (cols != o.cols) return cols < o.cols;
      return tokens < o.tokens;
    }
  };
  struct ProfStat {
    long long calls = 0;
    double us = 0.0, bytes = 0.0, ops = 0.0;
  };
  struct ProfPending {
    ProfKey key;
    double bytes, ops;
    hipEvent_t a, b;
  };
  bool prof_on = false;
  std::map<ProfKey, ProfStat> prof;
  std::vector<ProfPending> prof_pending;
  std::vector<hipEvent_t> prof_events;  // created and free for reuse
  long long prof_untimed = 0;
  char name[96] = "hip";
  char desc[512] = "";
};

static void memo_clear(qhip_backend* be) {
  be->memo_src = nullptr;
  be->memo_cols = be->memo_k = 0;
  be->memo_fam = -1;
}

static constexpr size_t kArenaChunk = size_t(1) << 30;  // 1 GiB
static constexpr size_t kAlign = 256;

static bool over_budget(const qhip_backend* be, size_t more) { return be->budget && be->placed + more > be->budget; }

static hipError_t budget_error(const qhip_backend* be, const char* what, size_t more) {
  fprintf(stderr,
          "qwen35_hip: %s needs %zu MiB more; this backend has placed %zu MiB of its %zu MiB device budget\n",
          what, more >> 20, be->placed >> 20, be->budget >> 20);
  return hipErrorOutOfMemory;
}

static hipError_t arena_alloc(qhip_backend* be, size_t bytes, uint8_t** out) {
  bytes = (bytes + kAlign - 1) / kAlign * kAlign;
  if (over_budget(be, bytes)) return budget_error(be, "weight upload", bytes);
  if (!be->arena.empty()) {
    auto& c = be->arena.back();
    if (c.size - c.used >= bytes) {
      *out = c.base + c.used;
      c.used += bytes;
      be->placed += bytes;
      return hipSuccess;
    }
  }
  // a chunk of 1 GiB, or what is left of the budget if that is less
  size_t sz = bytes > kArenaChunk ? bytes : kArenaChunk;
  if (be->budget && sz > be->budget - be->placed) sz = bytes > be->budget - be->placed ? bytes : be->budget - be->placed;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess) return e;
  be->arena.push_back({(uint8_t*)p, sz, bytes});
  be->placed += bytes;
  *out = (uint8_t*)p;
  return hipSuccess;
}

static bool capturing(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Give up a scratch buffer that is being replaced by a larger one: freed now,
// or kept until free_scratch / destroy when a graph captured earlier may
// still read or write it.
static void release_buffer(qhip_backend* be, void* p, size_t bytes) {
  if (!p) return;
  if (be->graph_seen) {
    be->retired.emplace_back(p, bytes);
    return;
  }
  (void)hipFree(p);
  be->placed -= bytes;
}

// The size a growing buffer takes: at least half again its old size, so a
// sequence of growing prefills keeps few retired buffers (their total stays
// below twice the live one); exactly `bytes` when the budget has no room for
// more.
static size_t grown_size(const qhip_backend* be, size_t cap, size_t bytes) {
  const size_t g = cap + cap / 2;
  if (g <= bytes) return bytes;
  return over_budget(be, be->graph_seen ? g : g - cap) ? bytes : g;
}

static hipError_t ensure_act(qhip_backend* be, size_t bytes) {
  if (be->act_cap >= bytes) return hipSuccess;
  if (over_budget(be, be->graph_seen ? bytes : bytes - be->act_cap))
    return budget_error(be, "activation scratch", bytes - be->act_cap);
  bytes = grown_size(be, be->act_cap, bytes);
  release_buffer(be, be->act, be->act_cap);
  be->act = nullptr;
  be->act_cap = 0;
  memo_clear(be);
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return e;
  be->act = (uint8_t*)p;
  be->act_cap = bytes;
  be->placed += bytes;
  return hipSuccess;
}

static hipError_t ensure_skwork(qhip_backend* be, size_t bytes) {
  if (be->skwork_cap >= bytes) return hipSuccess;
  if (over_budget(be, be->graph_seen ? bytes : bytes - be->skwork_cap))
    return budget_error(be, "split-K workspace", bytes - be->skwork_cap);
  bytes = grown_size(be, be->skwork_cap, bytes);
  release_buffer(be, be->skwork, be->skwork_cap);
  be->skwork = nullptr;
  be->skwork_cap = 0;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return e;
  // the counters start at zero; a fill kernel on the backend's stream orders
  // it before the first split launch
  e = launch_fill_zero(p, kSkCountBytes, be->stream);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return e;
  }
  be->skwork = (uint8_t*)p;
  be->skwork_cap = bytes;
  be->placed += bytes;
  return hipSuccess;
}

static constexpr int kImgMmq = 0, kImgFrag = 1;

// An MMQ image of a Q6_K weight: looked up, or built now when images are on,
// the budget allows it and the stream is not being captured (building
// allocates).  nullptr = run the MMQ on the GGUF bytes instead.
static void* image_for(qhip_backend* be, const void* wdev, int ttype, int rows, int cols, int kind,
                       hipError_t* err) {
  *err = hipSuccess;
  const qhip_backend::ImageKey key{wdev, ttype, rows, cols, kind};
  auto it = be->images.find(key);
  if (it != be->images.end()) return it->second.p;
  if (!be->images_on || capturing(be->stream)) return nullptr;
  const long n = kind == kImgFrag ? qhip_wd_image_bytes(ttype, rows, cols) : qhip_mmq_image_bytes(ttype, rows, cols);
  if (n <= 0 || over_budget(be, (size_t)n)) return nullptr;
  void* img = nullptr;
  hipError_t e = hipMalloc(&img, (size_t)n);
  if (e != hipSuccess) {
    *err = e;
    return nullptr;
  }
  const int rc = kind == kImgFrag ? qhip_launch_wd_prepare(ttype, wdev, rows, cols, img, be->stream)
                                  : qhip_launch_mmq_prepare(ttype, wdev, rows, cols, img, be->stream);
  if (rc) {
    (void)hipFree(img);
    *err = (hipError_t)rc;
    return nullptr;
  }
  be->images.emplace(key, qhip_backend::Image{img, (size_t)n});
  be->placed += (size_t)n;
  return img;
}

// Bytes per value of the widest activation family (Q8_K: 292/256), so one
// scratch serves every weight type.
static size_t act_bytes_for(int cols, int k) {
  const size_t c = (size_t)((cols + 255) / 256) * 256;
  return c / 256 * 292 * (size_t)k + 256;
}

// memo family of the split activation the GEMV image reads: kFamSplit plus
// its layout (gemv_image_layout; the other families are the activation
// block sizes, 32 and 256)
static constexpr int kFamSplit = 1 << 16;

static hipError_t img_arena_alloc(qhip_backend* be, size_t bytes, uint8_t** out) {
  bytes = (bytes + kAlign - 1) / kAlign * kAlign;
  if (over_budget(be, bytes)) return hipErrorOutOfMemory;
  if (!be->img_arena.empty()) {
    auto& c = be->img_arena.back();
    if (c.size - c.used >= bytes) {
      *out = c.base + c.used;
      c.used += bytes;
      be->placed += bytes;
      return hipSuccess;
    }
  }
  size_t sz = bytes > kArenaChunk ? bytes : kArenaChunk;
  if (be->budget && sz > be->budget - be->placed) sz = bytes;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, sz);
  if (e != hipSuccess) return e;
  be->img_arena.push_back({(uint8_t*)p, sz, bytes});
  be->placed += bytes;
  *out = (uint8_t*)p;
  return hipSuccess;
}

// The image bytes of GGUF rows [wdev, wdev + rows * row_bytes), when images
// cover them contiguously (one image, or adjacent images of adjacent
// weights); nullptr otherwise.
static uint8_t* gimage_lookup(const qhip_backend* be, const void* wdev, int ttype, int rows, int cols,
                              long row_bytes) {
  const uint8_t* p = (const uint8_t*)wdev;
  long need = rows;
  uint8_t* first = nullptr;
  uint8_t* expect = nullptr;
  while (need > 0) {
    auto it = be->gimages.upper_bound(p);
    if (it == be->gimages.begin()) return nullptr;
    --it;
    const qhip_backend::GImage& g = it->second;
    if (g.ttype != ttype || g.cols != cols || g.row_bytes != row_bytes) return nullptr;
    const long off = (long)(p - it->first);
    if (off % row_bytes || off / row_bytes >= g.rows) return nullptr;
    uint8_t* ip = g.img + off;
    if (first == nullptr) first = ip;
    else if (ip != expect) return nullptr;
    const long take = need < g.rows - off / row_bytes ? need : g.rows - off / row_bytes;
    need -= take;
    p += take * row_bytes;
    expect = ip + take * row_bytes;
  }
  return first;
}

// Build the image of rows [wdev, wdev + rows * row_bytes) when images are on,
// the budget allows it and the stream is not being captured (building
// allocates); nullptr = run the GGUF-layout path.
static uint8_t* gimage_for(qhip_backend* be, const void* wdev, int ttype, int rows, int cols, long row_bytes,
                           hipError_t* err) {
  *err = hipSuccess;
  if (uint8_t* hit = gimage_lookup(be, wdev, ttype, rows, cols, row_bytes)) return hit;
  if (!be->gemv_images_on || capturing(be->stream)) return nullptr;
  const long n = qhip_gemv_image_bytes(ttype, rows, cols);
  if (n <= 0 || over_budget(be, (size_t)n)) return nullptr;
  uint8_t* img = nullptr;
  hipError_t e = img_arena_alloc(be, (size_t)n, &img);
  if (e != hipSuccess) {
    if (e != hipErrorOutOfMemory) *err = e;
    return nullptr;
  }
  const int rc = qhip_launch_gemv_prepare(ttype, wdev, rows, cols, img, be->stream);
  if (rc) {
    *err = (hipError_t)rc;
    return nullptr;
  }
  be->gimages[(const uint8_t*)wdev] = qhip_backend::GImage{img, ttype, rows, cols, row_bytes};
  return img;
}

static int report(const char* what, hipError_t e) {
  if (e != hipSuccess && (int)e != QHIP_DECLINE)
    fprintf(stderr, "qwen35_hip: %s failed: %s\n", what, hipGetErrorString(e));
  return (int)e;
}

static bool valid_linear(const qhip_linear* w) {
  return w && w->dev && qhip_weight_row_bytes(w->ttype, w->cols) == w->row_bytes && w->rows >= 0;
}

// quantize `k` tokens of x into the scratch and run out = W . xq
static int run(qhip_backend* be, float* out, const void* wdev, int ttype, int rows, int cols,
               long row_bytes, const float* x, int k) {
  if (!out || !x || k < 0) return (int)hipErrorInvalidValue;
  if (k == 0 || rows == 0) return 0;
  if (!be->graph_seen && capturing(be->stream)) be->graph_seen = true;
  // the activation family: Q8_0 rows for 32-value weight blocks, Q8_K for
  // 256-value super-blocks (backend_cpu.zig:42-50 actFamily)
  const int fam = qhip_quant_act_block_elems(ttype);
  if (k == 1 && be->gemv_images_on) {
    // the 32-value 4-bit formats on larger matrices: split quantize + GEMV
    // from the weight's GEMV image
    const GemvArgs g1{ttype, wdev, x, out, rows, cols, 1, row_bytes, qhip_act_row_bytes(ttype, cols)};
    if (gemv_image_preferred(g1)) {
      hipError_t ei;
      uint8_t* img = gimage_for(be, wdev, ttype, rows, cols, row_bytes, &ei);
      if (ei != hipSuccess) return report("GEMV image", ei);
      if (img) {
        const int sfam = kFamSplit + gemv_image_layout(ttype, cols);
        const bool hs = be->memo_on && be->memo_src == x && be->memo_cols == cols && be->memo_k == 1 &&
                        be->memo_fam == sfam && be->act;
        if (be->memo_on) (hs ? be->memo_hits : be->memo_misses)++;
        if (!hs) {
          const hipError_t ea = ensure_act(be, act_bytes_for(cols, 1));
          if (ea != hipSuccess) return report("activation scratch", ea);
          memo_clear(be);
          const int rq = qhip_launch_quantize_act_image(ttype, x, be->act, cols, 1, be->stream);
          if (rq) return report("quantize", (hipError_t)rq);
          if (be->memo_on) {
            be->memo_src = x;
            be->memo_cols = cols;
            be->memo_k = 1;
            be->memo_fam = sfam;
          }
        }
        return report("matvec", (hipError_t)qhip_launch_mul_mat_vec_image(img, be->act, out, rows, cols, ttype, 0,
                                                                           be->stream));
      }
    }
  }
  // Q6_K at one token, quantized separately: the weight's K-quant GEMV image
  // (the same GEMV launch as the GGUF rows, reading the image), in place of
  // the one-launch split-K form
  uint8_t* kimg = nullptr;
  if (k == 1 && be->gemv_images_on) {
    const GemvArgs gk{ttype, wdev, x, out, rows, cols, 1, row_bytes, qhip_act_row_bytes(ttype, cols)};
    if (gemv_kimage_preferred(gk)) {
      hipError_t ei;
      kimg = gimage_for(be, wdev, ttype, rows, cols, row_bytes, &ei);
      if (ei != hipSuccess) return report("GEMV image", ei);
    }
  }
  const bool hit = be->memo_on && be->memo_src == x && be->memo_cols == cols && be->memo_k == k &&
                   be->memo_fam == fam && be->act;
  if (be->memo_on) (hit ? be->memo_hits : be->memo_misses)++;
  if (!hit && k == 1 && !kimg) {
    // one launch, the activation quantized inside the GEMV, where that is
    // faster than a separate quantize launch (widths up to 4096 whole; long
    // rows split over K); with the memo on, the launch also leaves the
    // quantized rows in the scratch
    const GemvArgs g1{ttype, wdev, x, out, rows, cols, 1, row_bytes, qhip_act_row_bytes(ttype, cols)};
    const bool split = gemv_splitk_preferred(g1);
    if (split || gemv_fused_preferred(g1)) {
      void* xq_out = nullptr;
      if (be->memo_on) {
        const hipError_t ea = ensure_act(be, act_bytes_for(cols, 1));
        if (ea != hipSuccess) return report("activation scratch", ea);
        memo_clear(be);
        xq_out = be->act;
      }
      int rc;
      if (split) {
        const long wb = gemv_splitk_work_bytes(rows, cols);
        const hipError_t ew = ensure_skwork(be, (size_t)wb);
        if (ew != hipSuccess) return report("split-K workspace", ew);
        rc = qhip_launch_quantize_mul_mat_vec_split(wdev, x, xq_out, out, rows, cols, ttype, 0, 0, 0, be->skwork,
                                                    (long)be->skwork_cap, be->stream);
      } else {
        rc = qhip_launch_quantize_mul_mat_vec(wdev, x, xq_out, out, rows, cols, ttype, be->stream);
      }
      if (rc != QHIP_DECLINE) {
        if (rc == 0 && xq_out) {
          be->memo_src = x;
          be->memo_cols = cols;
          be->memo_k = 1;
          be->memo_fam = fam;
        }
        return report("matvec", (hipError_t)rc);
      }
    }
  }
  hipError_t e = hipSuccess;
  int rc = 0;
  if (!hit) {
    e = ensure_act(be, act_bytes_for(cols, k));
    if (e != hipSuccess) return report("activation scratch", e);
    memo_clear(be);
    rc = qhip_launch_quantize_act(ttype, x, be->act, cols, k, be->stream);
    if (rc) return report("quantize", (hipError_t)rc);
    if (be->memo_on) {
      be->memo_src = x;
      be->memo_cols = cols;
      be->memo_k = k;
      be->memo_fam = fam;
    }
  }
  GemvArgs g{ttype, wdev, be->act, out, rows, cols, k, row_bytes, qhip_act_row_bytes(ttype, cols)};
  if (kimg) {
    GemvArgs gi = g;
    gi.w = kimg;
    gi.kimg = true;
    return report("matvec", launch_gemv(gi, 0, 0, 0, be->stream));
  }
  // the MMQ's split-K workspace for small grids, grown outside a capture
  // only (under capture a launch that does not fit runs unsplit)
  const long need = mul_mat_work_bytes(g);
  if (need > 0 && (size_t)need > be->skwork_cap && !capturing(be->stream)) {
    e = ensure_skwork(be, (size_t)need);
    if (e != hipSuccess && e != hipErrorOutOfMemory) return report("split-K workspace", e);
  }
  void* work = be->skwork;
  const long work_bytes = (long)be->skwork_cap;
  if (wd_image_preferred(g)) {
    // a few tokens of a Q6_K weight: the MMQ from its fragment image
    void* img = image_for(be, wdev, ttype, rows, cols, kImgFrag, &e);
    if (e != hipSuccess) return report("fragment image", e);
    if (img)
      return report("matvec", (hipError_t)qhip_launch_mul_mat_wd_image(img, be->act, out, rows, cols, k, ttype, work,
                                                                        work_bytes, be->stream));
  }
  if (mmq_image_preferred(g)) {
    // prefill of a Q6_K weight: MMQ from its image when there is one
    void* img = image_for(be, wdev, ttype, rows, cols, kImgMmq, &e);
    if (e != hipSuccess) return report("MMQ image", e);
    if (img)
      return report("matvec", (hipError_t)qhip_launch_mul_mat_image(img, be->act, out, rows, cols, k, ttype, 0, 0,
                                                                     work, work_bytes, be->stream));
  }
  return report("matvec", dispatch_mul_mat(g, QHIP_PATH_AUTO, work, work_bytes, be->stream));
}

// ---- device timing of the slots ---------------------------------------------------

static constexpr size_t kProfMaxPending = 512;
static const char* const kSlotNames[] = {"matvec", "matvecPair", "matvecBatchK", "dequantRow"};

static hipEvent_t prof_event(qhip_backend* be) {
  if (!be->prof_events.empty()) {
    hipEvent_t e = be->prof_events.back();
    be->prof_events.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

// Read the oldest recorded pairs (waiting for them) until `keep` remain.
static void prof_resolve(qhip_backend* be, size_t keep) {
  const size_t n = be->prof_pending.size() > keep ? be->prof_pending.size() - keep : 0;
  for (size_t i = 0; i < n; ++i) {
    qhip_backend::ProfPending& p = be->prof_pending[i];
    float ms = 0.0f;
    if (hipEventSynchronize(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
      qhip_backend::ProfStat& st = be->prof[p.key];
      st.calls += 1;
      st.us += 1e3 * (double)ms;
      st.bytes += p.bytes;
      st.ops += p.ops;
    }
    be->prof_events.push_back(p.a);
    be->prof_events.push_back(p.b);
  }
  be->prof_pending.erase(be->prof_pending.begin(), be->prof_pending.begin() + (long)n);
}

// One timed slot call: start() records the opening event, finish() the
// closing one and queues the pair with the call's algorithmic bytes
// (weights + f32 x + f32 y) and int8 ops (2 rows cols tokens).
struct ProfScope {
  qhip_backend* be;
  hipEvent_t a = nullptr;
  ProfScope(qhip_backend* b) : be(b) {
    if (!be->prof_on) return;
    if (capturing(be->stream)) {
      ++be->prof_untimed;
      return;
    }
    a = prof_event(be);
    if (a && hipEventRecord(a, be->stream) != hipSuccess) {
      be->prof_events.push_back(a);
      a = nullptr;
    }
  }
  int finish(int rc, int slot, int ttype, int rows, int cols, int tokens, double wbytes) {
    if (!a) return rc;
    hipEvent_t b = rc == 0 ? prof_event(be) : nullptr;
    if (!b || hipEventRecord(b, be->stream) != hipSuccess) {
      be->prof_events.push_back(a);
      if (b) be->prof_events.push_back(b);
      return rc;
    }
    const double bytes = slot == 3 ? wbytes + 4.0 * cols : wbytes + 4.0 * ((double)cols + rows) * tokens;
    const double ops = slot == 3 ? 0.0 : 2.0 * rows * (double)cols * tokens;
    be->prof_pending.push_back({{slot, ttype, rows, cols, tokens}, bytes, ops, a, b});
    if (be->prof_pending.size() >= kProfMaxPending) prof_resolve(be, kProfMaxPending / 2);
    return rc;
  }
};

static const char* type_name(int ttype) {
  switch (ttype) {
    case QHIP_TT_Q4_0: return "Q4_0";
    case QHIP_TT_Q4_1: return "Q4_1";
    case QHIP_TT_Q8_0: return "Q8_0";
    case QHIP_TT_Q2_K: return "Q2_K";
    case QHIP_TT_Q3_K: return "Q3_K";
    case QHIP_TT_Q4_K: return "Q4_K";
    case QHIP_TT_Q5_K: return "Q5_K";
    case QHIP_TT_Q6_K: return "Q6_K";
    case QHIP_TT_IQ3_XXS: return "IQ3_XXS";
    case QHIP_TT_IQ4_NL: return "IQ4_NL";
    case QHIP_TT_IQ3_S: return "IQ3_S";
    case QHIP_TT_IQ4_XS: return "IQ4_XS";
    default: return "?";
  }
}

extern "C" {

qhip_backend* qhip_backend_create(int device, int* err) {
  int rc = qhip_init(device);
  if (err) *err = rc;
  if (rc) return nullptr;
  qhip_backend* be = new (std::nothrow) qhip_backend();
  if (!be) {
    if (err) *err = (int)hipErrorOutOfMemory;
    return nullptr;
  }
  be->device = device;
  snprintf(be->name, sizeof be->name, "hip:%d %s", device, qhip_gpu_name());
  return be;
}

void qhip_backend_destroy(qhip_backend* be) {
  if (!be) return;
  (void)hipSetDevice(be->device);
  (void)hipDeviceSynchronize();
  prof_resolve(be, 0);
  for (hipEvent_t e : be->prof_events) (void)hipEventDestroy(e);
  qhip_backend_free_scratch(be);
  for (auto& kv : be->images) (void)hipFree(kv.second.p);
  for (auto& c : be->arena) (void)hipFree(c.base);
  for (auto& c : be->img_arena) (void)hipFree(c.base);
  delete be;
}

const char* qhip_backend_name(const qhip_backend* be) { return be ? be->name : ""; }

int qhip_backend_load_linear(qhip_backend* be, int ttype, int rows, int cols, const void* host,
                             qhip_linear* out) {
  const long rb = qhip_weight_row_bytes(ttype, cols);
  if (!be || !out || !host || rows < 0 || rb < 0) return (int)hipErrorInvalidValue;
  const size_t bytes = (size_t)rows * (size_t)rb;
  uint8_t* dev = nullptr;
  hipError_t e = arena_alloc(be, bytes ? bytes : 1, &dev);
  if (e != hipSuccess) return report("weight upload", e);
  e = hipMemcpy(dev, host, bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) return report("weight upload", e);
  *out = qhip_linear{dev, ttype, rows, cols, rb};
  return 0;
}

int qhip_backend_wrap_linear(qhip_backend* be, int ttype, int rows, int cols, const void* d_data,
                             qhip_linear* out) {
  const long rb = qhip_weight_row_bytes(ttype, cols);
  if (!be || !out || !d_data || rows < 0 || rb < 0) return (int)hipErrorInvalidValue;
  *out = qhip_linear{d_data, ttype, rows, cols, rb};
  return 0;
}

void qhip_backend_free_linear(qhip_backend* be, qhip_linear* w) {
  // Arena memory is returned at destroy; MMQ images built from this weight's
  // bytes are freed now; the handle is cleared so a stale use fails
  // validation.
  if (be && w && w->dev) {
    (void)hipStreamSynchronize(be->stream);
    for (auto it = be->images.begin(); it != be->images.end();) {
      if (it->first.dev == w->dev) {
        (void)hipFree(it->second.p);
        be->placed -= it->second.bytes;
        it = be->images.erase(it);
      } else {
        ++it;
      }
    }
    const uint8_t* lo = (const uint8_t*)w->dev;
    const uint8_t* hi = lo + (size_t)w->rows * (size_t)w->row_bytes;
    for (auto it = be->gimages.begin(); it != be->gimages.end();) {
      const uint8_t* a = it->first;
      const uint8_t* b = a + (size_t)it->second.rows * (size_t)it->second.row_bytes;
      if (a < hi && lo < b) it = be->gimages.erase(it);
      else ++it;
    }
  }
  if (w) *w = qhip_linear{nullptr, 0, 0, 0, 0};
}

int qhip_backend_prepare_linear(qhip_backend* be, const qhip_linear* w) {
  if (!be || !valid_linear(w)) return (int)hipErrorInvalidValue;
  // a long prefill: whether any token count would use an image for this weight
  const GemvArgs g1{w->ttype, w->dev, w->dev, nullptr, w->rows, w->cols, 1, w->row_bytes,
                    qhip_act_row_bytes(w->ttype, w->cols)};
  if (be->gemv_images_on && (gemv_image_preferred(g1) || gemv_kimage_preferred(g1))) {
    // a decode matvec: the GEMV image
    if (capturing(be->stream)) return (int)hipErrorStreamCaptureUnsupported;
    hipError_t e;
    const uint8_t* img = gimage_for(be, w->dev, w->ttype, w->rows, w->cols, w->row_bytes, &e);
    if (e != hipSuccess) return report("GEMV image", e);
    if (!img) return QHIP_DECLINE;
  }
  // a few tokens (the fragment image) and a long prefill (the MMQ image)
  int rc = 0;
  for (const int kind : {kImgFrag, kImgMmq}) {
    const GemvArgs g{w->ttype, w->dev, w->dev, nullptr, w->rows, w->cols, kind == kImgFrag ? 8 : 4096,
                     w->row_bytes, qhip_act_row_bytes(w->ttype, w->cols)};
    if (!(kind == kImgFrag ? wd_image_preferred(g) : mmq_image_preferred(g))) continue;
    if (capturing(be->stream)) return (int)hipErrorStreamCaptureUnsupported;
    hipError_t e;
    void* img = image_for(be, w->dev, w->ttype, w->rows, w->cols, kind, &e);
    if (e != hipSuccess) return report(kind == kImgFrag ? "fragment image" : "MMQ image", e);
    if (!img) rc = QHIP_DECLINE;
  }
  return rc;
}

int qhip_backend_set_mmq_images(qhip_backend* be, int on) {
  if (!be) return (int)hipErrorInvalidValue;
  be->images_on = on != 0;
  return 0;
}

int qhip_backend_set_gemv_images(qhip_backend* be, int on) {
  if (!be) return (int)hipErrorInvalidValue;
  be->gemv_images_on = on != 0;
  memo_clear(be);
  return 0;
}

int qhip_backend_set_mem_budget(qhip_backend* be, size_t bytes) {
  if (!be) return (int)hipErrorInvalidValue;
  be->budget = bytes;
  return 0;
}

size_t qhip_backend_mem_placed(const qhip_backend* be) { return be ? be->placed : 0; }

int qhip_backend_alloc_scratch(qhip_backend* be, int max_cols) {
  return qhip_backend_alloc_scratch_k(be, max_cols, 1);
}

int qhip_backend_alloc_scratch_k(qhip_backend* be, int max_cols, int k) {
  if (!be || max_cols <= 0 || k <= 0) return (int)hipErrorInvalidValue;
  return report("scratch", ensure_act(be, act_bytes_for(max_cols, k)));
}

void qhip_backend_free_scratch(qhip_backend* be) {
  if (!be) return;
  (void)hipDeviceSynchronize();
  if (be->act) (void)hipFree(be->act);
  be->placed -= be->act_cap;
  be->act = nullptr;
  be->act_cap = 0;
  memo_clear(be);
  if (be->skwork) (void)hipFree(be->skwork);
  be->placed -= be->skwork_cap;
  be->skwork = nullptr;
  be->skwork_cap = 0;
  for (auto& b : be->bufs) {
    (void)hipFree(b.first);
    be->placed -= b.second;
  }
  be->bufs.clear();
  for (auto& b : be->retired) {
    (void)hipFree(b.first);
    be->placed -= b.second;
  }
  be->retired.clear();
}

int qhip_backend_alloc_buf(qhip_backend* be, size_t len, float** d_out) {
  if (!be || !d_out) return (int)hipErrorInvalidValue;
  const size_t bytes = len ? len * sizeof(float) : sizeof(float);
  if (over_budget(be, bytes)) return (int)budget_error(be, "allocBuf", bytes);
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) return report("allocBuf", e);
  be->bufs.emplace_back(p, bytes);
  be->placed += bytes;
  *d_out = (float*)p;
  return 0;
}

static double weight_bytes(const qhip_linear* w) { return (double)w->rows * (double)w->row_bytes; }

int qhip_backend_matvec(qhip_backend* be, float* d_out, const qhip_linear* w, const float* d_x) {
  if (!be || !valid_linear(w)) return (int)hipErrorInvalidValue;
  ProfScope ps(be);
  const int rc = run(be, d_out, w->dev, w->ttype, w->rows, w->cols, w->row_bytes, d_x, 1);
  return ps.finish(rc, 0, w->ttype, w->rows, w->cols, 1, weight_bytes(w));
}

int qhip_backend_matvec_pair(qhip_backend* be, float* d_out, const qhip_linear* a,
                             const qhip_linear* b, const float* d_x) {
  if (!be || !valid_linear(a) || !valid_linear(b) || !d_out) return (int)hipErrorInvalidValue;
  const bool alike = a->ttype == b->ttype && a->rows == b->rows && a->cols == b->cols;
  const bool adjacent =
      alike && (const uint8_t*)a->dev + (size_t)a->rows * a->row_bytes == (const uint8_t*)b->dev;
  ProfScope ps(be);
  int rc;
  if (adjacent) {
    rc = run(be, d_out, a->dev, a->ttype, 2 * a->rows, a->cols, a->row_bytes, d_x, 1);
  } else {
    rc = run(be, d_out, a->dev, a->ttype, a->rows, a->cols, a->row_bytes, d_x, 1);
    if (rc == 0) rc = run(be, d_out + a->rows, b->dev, b->ttype, b->rows, b->cols, b->row_bytes, d_x, 1);
  }
  return ps.finish(rc, 1, a->ttype, a->rows + b->rows, a->cols, 1, weight_bytes(a) + weight_bytes(b));
}

int qhip_backend_matvec_batch_k(qhip_backend* be, float* d_out, const qhip_linear* w,
                                const float* d_xK, int k) {
  if (!be || !valid_linear(w)) return (int)hipErrorInvalidValue;
  ProfScope ps(be);
  const int rc = run(be, d_out, w->dev, w->ttype, w->rows, w->cols, w->row_bytes, d_xK, k);
  return ps.finish(rc, 2, w->ttype, w->rows, w->cols, k, weight_bytes(w));
}

int qhip_backend_dequant_row(qhip_backend* be, float* d_dst, const qhip_linear* w, int row) {
  if (!be || !valid_linear(w) || !d_dst || row < 0 || row >= w->rows) return (int)hipErrorInvalidValue;
  ProfScope ps(be);
  const int rc = report("dequantRow", (hipError_t)qhip_launch_dequantize_row(
                                          w->ttype, (const uint8_t*)w->dev + (size_t)row * w->row_bytes, d_dst,
                                          w->cols, be->stream));
  return ps.finish(rc, 3, w->ttype, 1, w->cols, 1, (double)w->row_bytes);
}

int qhip_backend_set_profiling(qhip_backend* be, int on) {
  if (!be) return (int)hipErrorInvalidValue;
  be->prof_on = on != 0;
  return 0;
}

void qhip_backend_prof_reset(qhip_backend* be) {
  if (!be) return;
  prof_resolve(be, 0);
  be->prof.clear();
  be->prof_untimed = 0;
}

// The table, largest device time first.
static std::vector<std::pair<qhip_backend::ProfKey, qhip_backend::ProfStat>> prof_sorted(qhip_backend* be) {
  prof_resolve(be, 0);
  std::vector<std::pair<qhip_backend::ProfKey, qhip_backend::ProfStat>> v(be->prof.begin(), be->prof.end());
  std::stable_sort(v.begin(), v.end(), [](const auto& x, const auto& y) { return x.second.us > y.second.us; });
  return v;
}

int qhip_backend_prof_entries(qhip_backend* be, qhip_prof_entry* out, int max_entries) {
  if (!be || max_entries < 0 || (max_entries > 0 && !out)) return (int)hipErrorInvalidValue;
  const auto v = prof_sorted(be);
  const int n = (int)v.size() < max_entries ? (int)v.size() : max_entries;
  for (int i = 0; i < n; ++i) {
    const auto& k = v[(size_t)i].first;
    const auto& st = v[(size_t)i].second;
    out[i] = qhip_prof_entry{k.slot, k.ttype, k.rows, k.cols, k.tokens, st.calls, st.us, st.bytes, st.ops};
  }
  return (int)v.size();
}

long long qhip_backend_prof_untimed(const qhip_backend* be) { return be ? be->prof_untimed : 0; }

long qhip_backend_prof_report(qhip_backend* be, char* buf, long len) {
  if (!be || len < 0 || (len > 0 && !buf)) return -1;
  const auto v = prof_sorted(be);
  std::string t;
  char line[320];
  double us = 0.0;
  long long calls = 0;
  for (const auto& e : v) {
    us += e.second.us;
    calls += e.second.calls;
  }
  snprintf(line, sizeof line, "HIP-PROF %s slots=%zu calls=%lld device_ms=%.3f untimed_under_capture=%lld\n",
           be->name, v.size(), calls, us / 1e3, be->prof_untimed);
  t += line;
  for (const auto& e : v) {
    const auto& k = e.first;
    const auto& st = e.second;
    const double avg = st.calls ? st.us / (double)st.calls : 0.0;
    const double gbs = st.us > 0 ? st.bytes / (st.us * 1e3) : 0.0;
    const double tops = st.us > 0 ? st.ops / (st.us * 1e6) : 0.0;
    snprintf(line, sizeof line,
             "HIP-PROF %-12s %-7s rows=%-7d cols=%-6d k=%-5d calls=%-7lld total_us=%-11.1f avg_us=%-9.2f "
             "GB/s=%-7.0f hbm=%4.1f%% TOP/s=%.1f\n",
             kSlotNames[k.slot], type_name(k.ttype), k.rows, k.cols, k.tokens, st.calls, st.us, avg, gbs,
             100.0 * gbs / 8000.0, tops);
    t += line;
  }
  if (len > 0) {
    const size_t n = t.size() < (size_t)len - 1 ? t.size() : (size_t)len - 1;
    memcpy(buf, t.data(), n);
    buf[n] = 0;
  }
  return (long)t.size();
}

const char* qhip_backend_describe(qhip_backend* be) {
  if (!be) return "";
  size_t weights = 0, gemv_img = 0, mmq_img = 0;
  for (const auto& c : be->arena) weights += c.used;
  for (const auto& c : be->img_arena) gemv_img += c.used;
  for (const auto& kv : be->images) mmq_img += kv.second.bytes;
  const size_t scratch = be->act_cap + be->skwork_cap;
  char budget[48] = "no cap";
  if (be->budget) snprintf(budget, sizeof budget, "%zu MiB", be->budget >> 20);
  snprintf(be->desc, sizeof be->desc,
           "%s, %d CUs; weights %zu MiB, GEMV images %zu MiB, MMQ images %zu MiB, scratch %zu MiB, "
           "placed %zu MiB (budget %s); GEMV images %s, MMQ images %s, activation memo %s, profiling %s",
           be->name, qhip_gpu_cu_count(), weights >> 20, gemv_img >> 20, mmq_img >> 20, scratch >> 20,
           be->placed >> 20, budget, be->gemv_images_on ? "on" : "off", be->images_on ? "on" : "off",
           be->memo_on ? "on" : "off", be->prof_on ? "on" : "off");
  return be->desc;
}

int qhip_backend_set_stream(qhip_backend* be, void* stream) {
  if (!be) return (int)hipErrorInvalidValue;
  if (be->stream != (hipStream_t)stream) {
    memo_clear(be);
    // the scratch and the split-K workspace are single buffers: the old
    // stream's launches finish before another stream may write them (a
    // stream under capture has nothing in flight to wait for)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(be->stream, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
      const hipError_t e = hipStreamSynchronize(be->stream);
      if (e != hipSuccess) return report("set_stream", e);
    }
  }
  be->stream = (hipStream_t)stream;
  return 0;
}

int qhip_backend_set_act_memo(qhip_backend* be, int on) {
  if (!be) return (int)hipErrorInvalidValue;
  be->memo_on = on != 0;
  memo_clear(be);
  return 0;
}

void qhip_backend_act_invalidate(qhip_backend* be) {
  if (be) memo_clear(be);
}

int qhip_backend_act_stats(const qhip_backend* be, unsigned long long* hits, unsigned long long* misses) {
  if (!be) return (int)hipErrorInvalidValue;
  if (hits) *hits = be->memo_hits;
  if (misses) *misses = be->memo_misses;
  return 0;
}

void qhip_backend_step_begin(qhip_backend* be, unsigned pos) {
  (void)pos;
  if (be) memo_clear(be);
}

void qhip_backend_step_end(qhip_backend* be) { (void)be; }

int qhip_backend_sync(qhip_backend* be) {
  if (!be) return (int)hipErrorInvalidValue;
  return report("sync", hipStreamSynchronize(be->stream));
}

}  // extern "C"
