// pkv_probe.hip -- streaming read of whole pages: the bandwidth reference a
// decode launch is compared against (no counterpart in the reference).
//
// Wave w of W reads pages [w*n/W, (w+1)*n/W) of a page-id list in order, every
// byte of each page (all KV heads) as 16-byte loads, 16 per lane in flight
// (16 KiB per wave), non-temporal like the decode kernel's tile loads, and
// folds them into one word per lane so that the loads cannot be dropped.  Given the pages a decode step's sequences hold, in
// block-table order, and the decode launch's wave count, it moves the step's
// KV bytes with nothing but the loads: what HBM delivers for that access
// pattern on this device.
#include "pkv_launch.h"

namespace pkv {

namespace {

typedef uint32_t u4v __attribute__((ext_vector_type(4)));

constexpr int kInFlight = 16;  // 16-byte loads per lane per step

__global__ __launch_bounds__(64) void read_probe_kernel(const uint8_t *__restrict__ pool, int64_t num_pages,
                                                        int64_t page_bytes, const int32_t *__restrict__ ids,
                                                        int64_t count, uint32_t *__restrict__ out) {
  const int lane = threadIdx.x;
  const int64_t w = blockIdx.x, nw = gridDim.x;
  const int64_t p0 = w * count / nw, p1 = (w + 1) * count / nw;
  const int64_t units = page_bytes / 16;  // the page format keeps pages a multiple of 16 bytes
  u4v acc = {0, 0, 0, 0};
  for (int64_t p = p0; p < p1; ++p) {
    const int id = ids[p];
    if (id < 0 || id >= num_pages) continue;
    const u4v *base = (const u4v *)(pool + (int64_t)id * page_bytes);
    for (int64_t u0 = 0; u0 < units; u0 += 64 * kInFlight) {
      u4v v[kInFlight];
#pragma unroll
      for (int k = 0; k < kInFlight; ++k) {
        const int64_t u = u0 + k * 64 + lane;
        v[k] = u < units ? __builtin_nontemporal_load(base + u) : u4v{0, 0, 0, 0};
      }
#pragma unroll
      for (int k = 0; k < kInFlight; ++k) acc ^= v[k];
    }
  }
  out[w * 64 + lane] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

}  // namespace

hipError_t launch_read_probe(hipStream_t stream, const uint8_t *pool, int64_t num_pages, int64_t page_bytes,
                             const int32_t *ids, int64_t count, int waves, uint32_t *out) {
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)waves), dim3(64), 0, stream, pool, num_pages,
                     page_bytes, ids, count, out);
  return hipGetLastError();
}

}  // namespace pkv
