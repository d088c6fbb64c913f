// Plain HBM streaming copy: the bandwidth ceiling the benchmark measures
// beside the datasheet peak, and the calibration kernel of the HBM byte
// counters.  Each thread moves four 16-byte vectors per step with
// non-temporal loads and stores (nothing is re-read, so nothing should stay in
// the caches), over a grid-stride loop; all loads of a step are issued before
// its stores.  No counterpart in the reference.
#include "gdn_common.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kThreads) void hbm_stream_copy_kernel(const u32x4* __restrict__ src,
                                                                   u32x4* __restrict__ dst, int64_t n) {
  const int64_t step = (int64_t)gridDim.x * kThreads * kUnroll;
  for (int64_t base = (int64_t)blockIdx.x * kThreads * kUnroll + threadIdx.x; base < n; base += step) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * kThreads;
      if (i < n) v[u] = __builtin_nontemporal_load(src + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + (int64_t)u * kThreads;
      if (i < n) __builtin_nontemporal_store(v[u], dst + i);
    }
  }
}

}  // namespace

hipError_t hbm_stream_copy_launch(const void* src, void* dst, int64_t nbytes, int32_t blocks, hipStream_t st) {
  const int64_t n = nbytes / 16;
  if (n == 0) return hipSuccess;
  const int64_t need = (n + kThreads * kUnroll - 1) / (kThreads * kUnroll);
  const int64_t grid = blocks > 0 ? (need < blocks ? need : blocks) : need;
  hbm_stream_copy_kernel<<<dim3((unsigned)grid), dim3(kThreads), 0, st>>>(reinterpret_cast<const u32x4*>(src),
                                                                          reinterpret_cast<u32x4*>(dst), n);
  return hipGetLastError();
}
