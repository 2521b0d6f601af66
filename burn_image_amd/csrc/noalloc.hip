// biq_q4_linear_noalloc: the packed-Q4 projection for callers that cannot allocate device memory
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// It runs exactly the kernels and the work split of biq_q4_linear, so its results are bitwise
// those of biq_q4_linear; only the scratch differs.  biq_q4_linear takes the partial sums of its
// K-split tail tiles and of the small-M route from the library's grow-only per-stream workspace
// (allocated on first use); this entry point takes them from `scratch`, a file-scope device array
// of BIQ_NOALLOC_SCRATCH_BYTES that every GPU running the library holds until the process ends.
// A call whose work split needs more is rejected (BIQ_ERR_UNSUPPORTED) before any GPU work.
// Every scratch element a reduction reads is first written by the same call, so nothing is
// cleared between calls.  All calls on one GPU share its array: calls that overlap on one GPU
// (different streams, or host threads without ordering) race.
#include <mutex>

#include "common.h"

namespace {

// Static scratch: 32 MiB holds the largest split of the 4608-token projections (QKV: 96 partial
// tiles of 128 KiB = 12 MiB), the 1024-row Qwen projections (up to 256 partial tiles = 32 MiB)
// and the small-M route's partial rows up to 16 x 9216 x 24 chunks (14 MiB).
constexpr size_t SCRATCH_BYTES = (size_t)32 << 20;
static_assert(SCRATCH_BYTES == BIQ_NOALLOC_SCRATCH_BYTES, "header and library disagree on the scratch size");

__device__ __align__(256) unsigned char scratch[SCRATCH_BYTES];

// Device address of `scratch` on each device, resolved once per device with that device current
// (each GPU holds its own copy of the array at its own address).  In host code `scratch` names a
// host-side stand-in, never the device memory: only these addresses reach kernels.
constexpr int MAX_DEVICES = 64;
std::mutex g_mutex;
void *g_scratch_ptr[MAX_DEVICES] = {};

int device_scratch(biq::Scratch *out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return biq::fail(BIQ_ERR_HIP, "no current HIP device");
  if (dev < 0 || dev >= MAX_DEVICES) return biq::fail(BIQ_ERR_UNSUPPORTED, "device index beyond 64");
  std::lock_guard<std::mutex> lock(g_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return biq::fail(BIQ_ERR_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  out->ptr = g_scratch_ptr[dev];
  out->bytes = SCRATCH_BYTES;
  return BIQ_OK;
}

}  // namespace

namespace biq {
int q4_linear_launch(void *stream, const void *x, int x_dtype, int64_t M, int64_t K, int64_t ldx,
                     const uint32_t *words, const float *scales, int layout, int block, int64_t N,
                     const float *bias, void *y, int y_dtype, const Scratch *scr);
}

extern "C" int biq_q4_linear_noalloc(void *stream, const void *x, int x_dtype, int64_t M, int64_t K,
                                     int64_t ldx, const uint32_t *words, const float *scales,
                                     int layout, int block, int64_t N, const float *bias, void *y,
                                     int y_dtype) {
  biq::clear_error();
  biq::Scratch scr{nullptr, 0};
  const int st = device_scratch(&scr);
  if (st != BIQ_OK) return st;
  return biq::q4_linear_launch(stream, x, x_dtype, M, K, ldx, words, scales, layout, block, N, bias, y,
                               y_dtype, &scr);
}
