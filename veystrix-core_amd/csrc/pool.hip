// Miss fill of the device-resident expert-pool LRU (gfx950): the missed
// records, read by the GPU straight from pinned host memory (the reads run at
// the rate of a DMA copy) and written into their slots, so the host neither
// waits for the routes nor drives a copy engine.  The assign that lists the
// misses is k_select_lru (decode.hip, vm_lru.h).

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "vm_internal.h"

namespace vm {

namespace {

constexpr int kFillThreads = 256;
constexpr int kFillBlocks = 128;  // 128 blocks of 4 loads in flight per thread saturate the host link

// The missed records of a call as one flat range of 16-byte units (record
// after record), so the loads of the next record are in flight while the last
// ones of the previous record land: copying records one by one drained the
// pipeline at every record end.  Each thread walks the range with a grid
// stride, four units per step, loads before stores.
__global__ __launch_bounds__(kFillThreads) void k_pool_fill(FillLaunch p) {
  __shared__ const uint8_t* s_src[kLruMaxRouted];
  __shared__ uint8_t* s_dst[kLruMaxRouted];
  const uint32_t M = min(*p.count, kLruMaxRouted);
  for (uint32_t m = threadIdx.x; m < M; m += kFillThreads) {
    const uint32_t src = p.src[m], dst = p.dst[m];
    const bool ok = src < p.host_records && dst < p.pool_records;
    s_src[m] = ok ? p.host + static_cast<uint64_t>(src) * p.host_stride : nullptr;
    s_dst[m] = ok ? p.pool + p.header + static_cast<uint64_t>(dst) * p.stride : nullptr;
  }
  __syncthreads();
  const uint32_t upr = static_cast<uint32_t>(p.record_bytes / 16);  // units per record
  const uint32_t total = M * upr;
  const uint32_t stride = gridDim.x * kFillThreads;
  uint32_t u = blockIdx.x * kFillThreads + threadIdx.x;
  uint32_t m = u / upr, off = u - m * upr;
  while (u < total) {
    const uint4* src[4];
    uint4* dst[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      src[k] = nullptr;
      dst[k] = nullptr;
      if (u < total && s_src[m] != nullptr) {
        src[k] = reinterpret_cast<const uint4*>(s_src[m]) + off;
        dst[k] = reinterpret_cast<uint4*>(s_dst[m]) + off;
      }
      u += stride;
      off += stride;
      while (off >= upr) {
        off -= upr;
        ++m;
      }
    }
    uint4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (src[k] != nullptr) v[k] = *src[k];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (dst[k] != nullptr) *dst[k] = v[k];
  }
}

template <class... KArgs, class... Args>
hipError_t launch(const char* family, void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream,
                  Args... args) {
  hipEvent_t start = nullptr, stop = nullptr;
  if (timing_events(family, &start, &stop))
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_fill(const FillLaunch& p, hipStream_t stream) {
  return launch("fill", k_pool_fill, dim3(kFillBlocks), dim3(kFillThreads), stream, p);
}

}  // namespace vm
