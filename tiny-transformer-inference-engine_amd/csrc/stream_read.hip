// Plain streaming read of a contiguous buffer: the calibration the benchmark
// sets beside the attention kernels (the HBM read rate this device reaches
// on a kernel that does nothing but read, for the same byte count). Every
// thread reads 16-byte vectors at a grid stride with non-temporal loads
// (the decode kernels' load type) and folds them into one word, which is
// stored only if it equals an impossible value, so the loads cannot be
// removed and nothing is written. No counterpart in the reference.
#include "pkv_internal.h"

namespace pkv {
namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kSrThreads = 256;

__global__ __launch_bounds__(kSrThreads) void stream_read_kernel(const u32x4* __restrict__ p,
                                                                 int64_t n16,
                                                                 unsigned* __restrict__ sink) {
  unsigned acc = 0;
  const int64_t stride = (int64_t)gridDim.x * kSrThreads;
  for (int64_t i = (int64_t)blockIdx.x * kSrThreads + threadIdx.x; i < n16; i += stride) {
    const u32x4 v = __builtin_nontemporal_load(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u && sink) sink[0] = acc;
}

}  // namespace
}  // namespace pkv

extern "C" int pkv_stream_read(const void* p, int64_t bytes, unsigned* sink, int grid,
                               void* stream) {
  using namespace pkv;
  if (!p || bytes < 0 || grid <= 0)
    return fail(PKV_ERR_INVALID, "stream_read: p=%p bytes=%lld grid=%d", p, (long long)bytes, grid);
  if ((reinterpret_cast<uintptr_t>(p) & 15) != 0 || (bytes & 15) != 0)
    return fail(PKV_ERR_INVALID, "stream_read: buffer and size must be 16-byte multiples");
  if (bytes == 0) return PKV_OK;
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(kSrThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(p), bytes / 16,
                     sink);
  return check_launch("stream_read_kernel");
}
