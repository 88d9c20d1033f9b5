// Greedy token selection: the index of the largest logit of every row, the
// step after the vocabulary projection in a greedy decode loop
// (serving/generation.py:77-142 takes logits.argmax per sequence; the
// reference's sampler, sampling.py:5-137, is greedy = argmax). Same result
// as the framework's argmax: the first index holding the maximum, and a NaN
// counts as larger than every number (the first NaN wins).
//
// One workgroup per row streams it once with 16-byte loads (a scalar head
// up to the first 16-byte boundary, since rows of an odd vocabulary start
// unaligned, then vectors, then a scalar tail), keeping per thread the best
// (value, index); the candidates are combined across the wavefront by lane
// swaps and across wavefronts through LDS with the same ordering rule.
#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kAmThreads = 512;
constexpr int kAmWaves = kAmThreads / 64;
constexpr int kAmUnroll = 4;

// (v, i) precedes (bv, bi) in argmax order
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  const bool vn = v != v;
  const bool bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

template <typename T>
__global__ __launch_bounds__(kAmThreads) void argmax_rows_kernel(int64_t* __restrict__ ids,
                                                                 const T* __restrict__ logits,
                                                                 int64_t row_stride, int vocab) {
  constexpr int V = 16 / sizeof(T);
  const T* row = logits + (int64_t)blockIdx.x * row_stride;
  const int tid = threadIdx.x;
  float best = -INFINITY;
  int bi = 0x7fffffff;

  // elements before the first 16-byte boundary
  const int head = min(vocab, (int)(((16 - ((uintptr_t)row & 15)) & 15) / sizeof(T)));
  if (tid < head) {
    best = (float)row[tid];
    bi = tid;
  }
  const int nvec = (vocab - head) / V;
  const T* vrow = row + head;
  // vectors: thread tid takes vectors tid, tid + 512, ... (indices increase
  // along a thread's sequence, so a strict > keeps the first maximum)
  for (int v0 = tid; v0 < nvec; v0 += kAmThreads * kAmUnroll) {
    uint4 raw[kAmUnroll];
#pragma unroll
    for (int u = 0; u < kAmUnroll; ++u) {
      const int vv = v0 + u * kAmThreads;
      raw[u] = vv < nvec ? *reinterpret_cast<const uint4*>(vrow + (int64_t)vv * V)
                         : uint4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kAmUnroll; ++u) {
      const int vv = v0 + u * kAmThreads;
      if (vv >= nvec) break;
      T e[V];
      __builtin_memcpy(e, &raw[u], 16);
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const float x = (float)e[j];
        const int ix = head + vv * V + j;
        if (better(x, ix, best, bi)) {
          best = x;
          bi = ix;
        }
      }
    }
  }
  // tail
  for (int ix = head + nvec * V + tid; ix < vocab; ix += kAmThreads) {
    const float x = (float)row[ix];
    if (better(x, ix, best, bi)) {
      best = x;
      bi = ix;
    }
  }
  // combine: wavefront, then workgroup
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(best, o);
    const int oi = __shfl_xor(bi, o);
    if (better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  __shared__ float s_v[kAmWaves];
  __shared__ int s_i[kAmWaves];
  if ((tid & 63) == 0) {
    s_v[tid >> 6] = best;
    s_i[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kAmWaves; ++w)
      if (better(s_v[w], s_i[w], best, bi)) {
        best = s_v[w];
        bi = s_i[w];
      }
    ids[blockIdx.x] = bi;
  }
}

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" {

int pkv_argmax_rows(int64_t* ids, const void* logits, int64_t rows, int64_t vocab,
                    int64_t row_stride, int dtype, void* stream) {
  if (dtype != PKV_DTYPE_F32 && dtype != PKV_DTYPE_F16 && dtype != PKV_DTYPE_BF16)
    return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  if (rows < 0 || vocab <= 0 || vocab > 0x7fffffff || row_stride < vocab)
    return fail(PKV_ERR_INVALID, "argmax_rows: bad sizes rows=%lld vocab=%lld stride=%lld",
                (long long)rows, (long long)vocab, (long long)row_stride);
  if (rows > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "argmax_rows: %lld rows", (long long)rows);
  if (!ids || !logits) return fail(PKV_ERR_INVALID, "null pointer argument");
  if (((uintptr_t)logits % elem_bytes(dtype)) != 0)
    return fail(PKV_ERR_INVALID, "argmax_rows: logits not aligned to the element size");
  if (rows == 0) return PKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)rows), block(kAmThreads);
  if (dtype == PKV_DTYPE_BF16)
    hipLaunchKernelGGL((argmax_rows_kernel<bf16>), grid, block, 0, s, ids,
                       static_cast<const bf16*>(logits), row_stride, (int)vocab);
  else if (dtype == PKV_DTYPE_F16)
    hipLaunchKernelGGL((argmax_rows_kernel<f16>), grid, block, 0, s, ids,
                       static_cast<const f16*>(logits), row_stride, (int)vocab);
  else
    hipLaunchKernelGGL((argmax_rows_kernel<float>), grid, block, 0, s, ids,
                       static_cast<const float*>(logits), row_stride, (int)vocab);
  return check_launch("argmax_rows_kernel");
}

}  // extern "C"
