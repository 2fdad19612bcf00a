// TOPK-32 of the LM head for gfx950 as a kernel of its own, over a y32
// vector already in memory: one wavefront per chunk of the scan in
// w4a8_topk_device.h (1024 rows; the first 256), the chunks in parallel.
// Workgroups are dispatched in chunk order and a chunk only waits for
// lower-numbered chunks, which publish before they wait, so the waits
// cannot deadlock.
#include "w4a8_topk_device.h"

namespace w4a8 {

namespace {

using namespace tk;

// Chunk c = workgroup c.  Bit 3 of err: a wait gave up.
__global__ __launch_bounds__(64) void topk_kernel(const int32_t *y, int64_t n, int nchunks,
                                                  int32_t epoch, uint64_t *part, uint64_t *sup,
                                                  int32_t *flags, int32_t *out, int32_t *err,
                                                  uint32_t spin) {
  __shared__ uint64_t buf[128];
  __shared__ int32_t rows[kTkRows];
  const int lane = threadIdx.x;
  const int c = blockIdx.x;
  const bool up = tk_ror4_up();
  const int64_t s0 = chunk_first(c), end = chunk_end(c, n);
  int32_t yv[kTkPerLane];   // rows s0 + lane + 64 t, loads all in flight
#pragma unroll
  for (int t = 0; t < kTkPerLane; ++t) {
    const int64_t r = s0 + lane + 64 * t;
    yv[t] = r < end ? y[r] : 0;
  }
  const bool ok =
      chunk_run(yv, rows, buf, n, nchunks, c, epoch, part, sup, flags, out, spin, up, lane);
  if (!ok && lane == 0) atomicOr(err, 8);
}

}  // namespace

int topk_chunks(int64_t n) {
  using namespace tk;
  return n <= kTkFirst ? 1 : 1 + (int)((n - kTkFirst + kTkRows - 1) / kTkRows);
}

size_t topk_scratch_bytes(int64_t n) {
  return (size_t)(topk_chunks(n) + kTopkMaxChunks / kTopkSuper) * tk::kTk * 8;
}

hipError_t launch_topk32(const int32_t *y, int64_t n, void *scratch, int32_t *flags,
                         int32_t epoch, int32_t *out, int32_t *err, hipStream_t s,
                         uint32_t spin) {
  const int nchunks = topk_chunks(n);
  if (nchunks > kTopkMaxChunks) return hipErrorInvalidValue;
  uint64_t *part = (uint64_t *)scratch;
  hipLaunchKernelGGL(topk_kernel, dim3(nchunks), dim3(64), 0, s, y, n, nchunks, epoch, part,
                     part + (size_t)nchunks * tk::kTk, flags, out, err,
                     spin ? spin : tk::kTkSpin);
  return hipGetLastError();
}

}  // namespace w4a8
