// C ABI plumbing of libbiq: version, thread-local error state and the Q4S storage contract
// (host-only helpers that need no GPU).
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "common.h"

namespace biq {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }
int fail(int status, const std::string &msg) {
  g_last_error = msg;
  return status;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(BIQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
  return BIQ_OK;
}

// One grow-only scratch buffer per (device, stream): calls on one stream run in order, so they
// may share it; calls on different streams never do.  A buffer that is outgrown is kept, not
// freed (a captured graph may still name it); all of them live until the process ends or
// biq_release_stream_workspace releases the stream's buffers.
static std::mutex g_ws_mutex;
static std::map<std::pair<int, uintptr_t>, std::pair<void *, size_t>> g_ws;
static std::map<std::pair<int, uintptr_t>, std::vector<void *>> g_ws_outgrown;

int stream_workspace(hipStream_t s, size_t bytes, void **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(BIQ_ERR_HIP, "workspace: no current device");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  auto &e = g_ws[{dev, reinterpret_cast<uintptr_t>(s)}];
  if (e.first != nullptr && e.second >= bytes) {
    *out = e.first;
    return BIQ_OK;
  }
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(BIQ_ERR_UNSUPPORTED,
                "split-K workspace must grow outside stream capture: make the same call once before capturing");
  size_t want = bytes > 2 * e.second ? bytes : 2 * e.second;
  want = (want + (1u << 20) - 1) & ~((size_t)(1u << 20) - 1);
  void *p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess) return fail(BIQ_ERR_HIP, "workspace: hipMalloc failed");
  if (e.first != nullptr) g_ws_outgrown[{dev, reinterpret_cast<uintptr_t>(s)}].push_back(e.first);
  e = {p, want};
  *out = p;
  return BIQ_OK;
}

int get_scratch(hipStream_t s, const Scratch *fixed, size_t bytes, void **out) {
  if (fixed == nullptr) return stream_workspace(s, bytes, out);
  if (bytes > fixed->bytes)
    return fail(BIQ_ERR_UNSUPPORTED, "this call needs " + std::to_string(bytes) +
                                         " bytes of scratch; the static scratch holds " +
                                         std::to_string(fixed->bytes));
  *out = fixed->ptr;
  return BIQ_OK;
}

int device_cu_count() {
  static std::mutex m;
  static std::map<int, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(m);
  auto it = cache.find(dev);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
  cache[dev] = n;
  return n;
}

int release_stream_workspace(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(BIQ_ERR_HIP, "workspace: no current device");
  if (hipStreamSynchronize(s) != hipSuccess) return fail(BIQ_ERR_HIP, "workspace: stream synchronisation failed");
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  const std::pair<int, uintptr_t> key{dev, reinterpret_cast<uintptr_t>(s)};
  int st = BIQ_OK;
  auto it = g_ws.find(key);
  if (it != g_ws.end()) {
    if (hipFree(it->second.first) != hipSuccess) st = fail(BIQ_ERR_HIP, "workspace: hipFree failed");
    g_ws.erase(it);
  }
  auto old = g_ws_outgrown.find(key);
  if (old != g_ws_outgrown.end()) {
    for (void *p : old->second)
      if (hipFree(p) != hipSuccess) st = fail(BIQ_ERR_HIP, "workspace: hipFree failed");
    g_ws_outgrown.erase(old);
  }
  return st;
}

}  // namespace biq

extern "C" {

// Frees the scratch kept for (current device, stream) after waiting for the stream.
int biq_release_stream_workspace(void *stream) {
  biq::clear_error();
  return biq::release_stream_workspace(reinterpret_cast<hipStream_t>(stream));
}

const char *biq_version(void) { return "biq 0.1.0 gfx950"; }

const char *biq_last_error(void) { return biq::g_last_error.c_str(); }

// q4s_storage_block_and_axis (crates/burn_boogu/src/artifacts.rs:513-525).
int biq_q4_storage_block(int layout, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  if (layout == BIQ_Q4_NK_AXIS0) return cols % 128 == 0 ? 128 : 0;
  if (layout == BIQ_Q4_KN_AXIS1) {
    if (cols % 8 != 0) return 0;
    static const int groups[5] = {128, 64, 32, 16, 8};
    for (int g : groups)
      if (rows % g == 0) return g;
  }
  return 0;
}

// q4s_stored_dtype (artifacts.rs:527-536).
int biq_q4_stored_dtype(int layout, int64_t rows, int64_t cols, char *buf, size_t buf_len) {
  biq::clear_error();
  int block = biq_q4_storage_block(layout, rows, cols);
  if (block == 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, "shape has no exact Q4S storage contract");
  char tmp[64];
  if (layout == BIQ_Q4_NK_AXIS0)
    snprintf(tmp, sizeof tmp, "q4s-block%d-f32-packed-axis0", block);
  else
    snprintf(tmp, sizeof tmp, "q4s-block%dx1-f32-packed-axis1", block);
  if (buf == nullptr || buf_len <= strlen(tmp))
    return biq::fail(BIQ_ERR_INVALID_ARG, "stored dtype buffer too small");
  memcpy(buf, tmp, strlen(tmp) + 1);
  return BIQ_OK;
}

// Q4S tensor payload (the importer's single byte buffer: packed words, then f32 scales;
// crates/burn_boogu/src/artifacts.rs:7276-7283,7364-7377) -> layout, block and byte split, after
// checking the stored-dtype string and the size against the storage contract of the logical
// shape (q4s_stored_dtype, artifacts.rs:513-536; boogu_import.rs:1693-1719).
int biq_q4_payload_layout(const char *stored_dtype, int64_t rows, int64_t cols, int64_t payload_bytes,
                          int *layout, int *block, int64_t *words_bytes, int64_t *scales_bytes) {
  biq::clear_error();
  if (!stored_dtype || !layout || !block || !words_bytes || !scales_bytes)
    return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  int lay = -1;
  if (strstr(stored_dtype, "-packed-axis0") != nullptr) lay = BIQ_Q4_NK_AXIS0;
  else if (strstr(stored_dtype, "-packed-axis1") != nullptr) lay = BIQ_Q4_KN_AXIS1;
  if (lay < 0 || strncmp(stored_dtype, "q4s-block", 9) != 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, std::string("not a Q4S stored dtype: ") + stored_dtype);
  char expect[64];
  if (biq_q4_stored_dtype(lay, rows, cols, expect, sizeof expect) != BIQ_OK)
    return biq::fail(BIQ_ERR_INVALID_ARG, "the logical shape has no Q4S storage contract for this layout");
  if (strcmp(expect, stored_dtype) != 0)
    return biq::fail(BIQ_ERR_INVALID_ARG, std::string("stored dtype ") + stored_dtype + " does not match " +
                                              expect + " for this shape");
  const int blk = biq_q4_storage_block(lay, rows, cols);
  // logical [K, N] (axis 1) or [N, K] (axis 0); K is the packed and blocked axis
  const int64_t K = lay == BIQ_Q4_KN_AXIS1 ? rows : cols;
  const int64_t N = lay == BIQ_Q4_KN_AXIS1 ? cols : rows;
  const int64_t wb = K * N / 2, sb = (K / blk) * N * 4;
  if (payload_bytes != wb + sb)
    return biq::fail(BIQ_ERR_INVALID_ARG, "Q4S payload is " + std::to_string(payload_bytes) +
                                              " bytes; the contract needs " + std::to_string(wb + sb));
  *layout = lay;
  *block = blk;
  *words_bytes = wb;
  *scales_bytes = sb;
  return BIQ_OK;
}

// Host-side check of a packed sequence's segment table (the device kernel clamps whatever it reads,
// but only a valid table gives the per-frame result).
int biq_check_cu_seqlens(const int32_t *cu, int64_t nseg, int64_t S) {
  biq::clear_error();
  if (!cu) return biq::fail(BIQ_ERR_INVALID_ARG, "cu_seqlens is null");
  if (nseg <= 0) return biq::fail(BIQ_ERR_INVALID_ARG, "segment mask requires at least one segment");
  if (cu[0] != 0) return biq::fail(BIQ_ERR_INVALID_ARG, "cu_seqlens must start at 0");
  for (int64_t i = 0; i < nseg; ++i)
    if (cu[i + 1] <= cu[i])
      return biq::fail(BIQ_ERR_INVALID_ARG, "cu_seqlens must be strictly ascending (no empty segment)");
  if ((int64_t)cu[nseg] != S)
    return biq::fail(BIQ_ERR_INVALID_ARG, "cu_seqlens must end at the sequence length");
  return BIQ_OK;
}

// Qwen vision frame ranges (crates/burn_qwen3_vl/src/vision.rs:319-386: `frame_ranges:
// &[(usize, usize)]`, each frame attends within itself, outputs concatenated in frame order)
// -> the block-diagonal segment table.  The frames must tile [0, S) in order, each non-empty.
int biq_frame_ranges_to_cu_seqlens(const int64_t *ranges, int64_t nframes, int64_t S, int32_t *cu) {
  biq::clear_error();
  if (!ranges || !cu) return biq::fail(BIQ_ERR_INVALID_ARG, "null pointer argument");
  if (nframes <= 0) return biq::fail(BIQ_ERR_INVALID_ARG, "at least one frame is required");
  if (S <= 0 || S > 0x7fffffffLL) return biq::fail(BIQ_ERR_INVALID_ARG, "sequence length out of range");
  int64_t expect = 0;
  for (int64_t f = 0; f < nframes; ++f) {
    const int64_t a = ranges[2 * f], e = ranges[2 * f + 1];
    if (a != expect) return biq::fail(BIQ_ERR_INVALID_ARG, "frame ranges must be contiguous and start at 0");
    if (e <= a) return biq::fail(BIQ_ERR_INVALID_ARG, "frame ranges must be non-empty");
    if (e > S) return biq::fail(BIQ_ERR_INVALID_ARG, "frame range exceeds the sequence");
    expect = e;
  }
  if (expect != S) return biq::fail(BIQ_ERR_INVALID_ARG, "frame ranges must cover the sequence");
  cu[0] = 0;
  for (int64_t f = 0; f < nframes; ++f) cu[f + 1] = (int32_t)ranges[2 * f + 1];
  return BIQ_OK;
}

}  // extern "C"
