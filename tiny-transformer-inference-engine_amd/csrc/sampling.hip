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
#include <type_traits>

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


// ---- top-k / top-p sampling (sampling.py:5-137's sample(): temperature,
// apply_top_k, apply_top_p, softmax, one multinomial draw; the reference's
// top-k kernel, kernels/cuda-kSAMPLING/ksampling_kernel.cu:61-185, covers
// the top-k step alone). One workgroup per row:
//   1. y = x / temperature (fp32, correctly rounded), the row's finiteness,
//      and each thread's maximum;
//   2. t0 = the k-th largest of the 256 thread maxima: at least k values of
//      the row are >= t0, so every value of the top-k set is;
//   3. the values >= t0 (normally k to a few k of them) are collected in
//      LDS and sorted descending (ties by ascending index): the k-th is the
//      top-k threshold, and the survivors (every value >= it, ties kept, as
//      apply_top_k's `logits < kth` mask keeps them) are a prefix;
//   4. one wavefront takes the softmax over the survivors, the cumulative
//      mass in that order, keeps the prefix whose mass before each token is
//      at most top_p (the first always), renormalises, and picks the token
//      by inverse CDF in vocabulary order: the first kept index (ascending)
//      whose cumulative probability exceeds u * total, u the row's uniform.
// More than kSmpCand values >= t0 (only with massive ties) sets
// PKV_STATUS_SAMPLE_OVERFLOW and writes -1: the caller samples that call
// another way. A non-finite logit sets PKV_STATUS_NONFINITE, a non-finite
// scaled value (temperature underflow) PKV_STATUS_BAD_DISTRIBUTION.
constexpr int kSmpThreads = 256;
constexpr int kSmpCand = 1024;
constexpr int kSmpUnroll = 16;

// (ka, ia) comes before (kb, ib): larger value first, then smaller index
__device__ __forceinline__ bool smp_before(float ka, int ia, float kb, int ib) {
  return ka > kb || (ka == kb && ia < ib);
}

// descending bitonic sort of n (a power of two <= kSmpCand) LDS pairs
__device__ void smp_sort(float* key, int* idx, int n) {
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int p = threadIdx.x; p < (n >> 1); p += kSmpThreads) {
        const int i = 2 * p - (p & (stride - 1));
        const int j = i + stride;
        const float ki = key[i], kj = key[j];
        const int ii = idx[i], ij = idx[j];
        const bool swap = (i & size) == 0 ? smp_before(kj, ij, ki, ii) : smp_before(ki, ii, kj, ij);
        if (swap) {
          key[i] = kj;
          key[j] = ki;
          idx[i] = ij;
          idx[j] = ii;
        }
      }
    }
  }
  __syncthreads();
}

__device__ __forceinline__ float smp_wave_sum(float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <typename T>
__global__ __launch_bounds__(kSmpThreads) void sample_rows_kernel(
    int64_t* __restrict__ ids, const T* __restrict__ logits, int64_t row_stride, int vocab,
    float temperature, int top_k, float top_p, const float* __restrict__ uniforms,
    int* __restrict__ status) {
  __shared__ float key[kSmpCand];
  __shared__ int idx[kSmpCand];
  __shared__ int s_cnt, s_flags;
  const int tid = threadIdx.x;
  const T* row = logits + (int64_t)blockIdx.x * row_stride;
  if (tid == 0) {
    s_cnt = 0;
    s_flags = 0;
  }
  // 1. thread maxima and finiteness
  // (kSmpUnroll loads of a thread in flight together, indices past the row
  // clamped onto its last element; the arithmetic is branch-free so the
  // compiler can interleave the elements' division chains; temperature 1
  // divides exactly by skipping the division)
  float mx = -INFINITY;
  int flags = 0;
  auto pass1 = [&](auto unit) {
    for (int j0 = tid; j0 < vocab; j0 += kSmpUnroll * kSmpThreads) {
      float xv[kSmpUnroll];
#pragma unroll
      for (int q = 0; q < kSmpUnroll; ++q) xv[q] = (float)row[min(j0 + q * kSmpThreads, vocab - 1)];
#pragma unroll
      for (int q = 0; q < kSmpUnroll; ++q) {
        const bool in = j0 + q * kSmpThreads < vocab;
        const float y = decltype(unit)::value ? xv[q] : xv[q] / temperature;
        flags |= (in && !isfinite(xv[q])) ? PKV_STATUS_NONFINITE : 0;
        flags |= (in && isfinite(xv[q]) && !isfinite(y)) ? PKV_STATUS_BAD_DISTRIBUTION : 0;
        mx = in ? fmaxf(mx, y) : mx;
      }
    }
  };
  const bool unit_temp = temperature == 1.f;
  if (unit_temp)
    pass1(std::integral_constant<bool, true>{});
  else
    pass1(std::integral_constant<bool, false>{});
  key[tid] = mx;
  idx[tid] = tid;
  __syncthreads();
  if (flags) atomicOr(&s_flags, flags);
  // 2. t0 = the k-th largest thread maximum
  const int k = top_k < vocab ? top_k : vocab;
  smp_sort(key, idx, kSmpThreads);
  const float t0 = key[k - 1];
  __syncthreads();  // key / idx are reused below
  if (s_flags) {
    if (tid == 0) {
      ids[blockIdx.x] = -1;
      if (status) atomicOr(status, s_flags);
    }
    return;
  }
  // 3. candidates >= t0, sorted
  auto pass2 = [&](auto unit) {
    for (int j0 = tid; j0 < vocab; j0 += kSmpUnroll * kSmpThreads) {
      float yv[kSmpUnroll];
#pragma unroll
      for (int q = 0; q < kSmpUnroll; ++q) yv[q] = (float)row[min(j0 + q * kSmpThreads, vocab - 1)];
#pragma unroll
      for (int q = 0; q < kSmpUnroll; ++q)
        if (!decltype(unit)::value) yv[q] = yv[q] / temperature;
      unsigned hit = 0;
#pragma unroll
      for (int q = 0; q < kSmpUnroll; ++q)
        hit |= (j0 + q * kSmpThreads < vocab && yv[q] >= t0) ? 1u << q : 0u;
      while (hit) {  // rare: the few values >= t0
        const int q = __builtin_ctz(hit);
        hit &= hit - 1;
        float y = yv[0];
#pragma unroll
        for (int r = 1; r < kSmpUnroll; ++r) y = r == q ? yv[r] : y;
        const int at = atomicAdd(&s_cnt, 1);
        if (at < kSmpCand) {
          key[at] = y;
          idx[at] = j0 + q * kSmpThreads;
        }
      }
    }
  };
  if (unit_temp)
    pass2(std::integral_constant<bool, true>{});
  else
    pass2(std::integral_constant<bool, false>{});
  __syncthreads();
  const int nc = s_cnt;
  if (nc > kSmpCand) {
    if (tid == 0) {
      ids[blockIdx.x] = -1;
      if (status) atomicOr(status, PKV_STATUS_SAMPLE_OVERFLOW);
    }
    return;
  }
  int n = 64;
  while (n < nc) n <<= 1;
  for (int i = nc + tid; i < n; i += kSmpThreads) {
    key[i] = -INFINITY;
    idx[i] = 0x7fffffff;
  }
  smp_sort(key, idx, n);
  // 4. one wavefront: survivors, softmax, top-p prefix, inverse CDF
  if (tid >= 64) return;
  const int lane = tid;
  const float tk = key[k - 1];
  constexpr int PER = kSmpCand / 64;  // consecutive sorted positions per lane
  const int i0 = lane * PER;
  int ns_l = 0;
#pragma unroll
  for (int e = 0; e < PER; ++e) ns_l += (i0 + e < nc && key[i0 + e] >= tk) ? 1 : 0;
  int ns = ns_l;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ns += __shfl_xor(ns, off, 64);
  const float m = key[0];
  float ev[PER];
  float zl = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    ev[e] = i0 + e < ns ? expf(key[i0 + e] - m) : 0.f;
    zl += ev[e];
  }
  const float z = smp_wave_sum(zl);
  // cumulative probability in sorted order: lane prefix of the segment sums
  float pl = 0.f;
  float pv[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    pv[e] = ev[e] / z;
    pl += pv[e];
  }
  float incl = pl;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  float cum = incl - pl;  // mass before this lane's first element
  int keep_l = 0;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int i = i0 + e;
    if (i < ns && (i == 0 || cum <= top_p)) ++keep_l;
    cum += pv[e];
  }
  int nk = keep_l;
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) nk += __shfl_xor(nk, off, 64);
  // renormalised probabilities of the kept prefix
  float zk_l = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) zk_l += i0 + e < nk ? ev[e] : 0.f;
  const float zk = smp_wave_sum(zk_l);
  float tot_l = 0.f;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    pv[e] = i0 + e < nk ? ev[e] / zk : 0.f;
    tot_l += pv[e];
  }
  const float target = uniforms[blockIdx.x] * smp_wave_sum(tot_l);
  // inverse CDF in vocabulary order: token i's cumulative start is the sum
  // of the kept probabilities of smaller indices. The probabilities replace
  // the values in LDS (this wavefront's LDS accesses complete in order), and
  // the kept tokens are spread over the lanes.
#pragma unroll
  for (int e = 0; e < PER; ++e)
    if (i0 + e < nk) key[i0 + e] = pv[e];
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  int pick = 0x7fffffff, last = -1;
  for (int i = lane; i < nk; i += 64) {
    const int my = idx[i];
    float c = 0.f;
    for (int j = 0; j < nk; ++j) c += idx[j] < my ? key[j] : 0.f;
    if (c + key[i] > target) pick = min(pick, my);
    last = max(last, my);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    pick = min(pick, __shfl_xor(pick, off, 64));
    last = max(last, __shfl_xor(last, off, 64));
  }
  if (lane == 0) ids[blockIdx.x] = pick != 0x7fffffff ? pick : last;
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

int pkv_sample_rows(int64_t* ids, const void* logits, int64_t rows, int64_t vocab,
                    int64_t row_stride, float temperature, int top_k, float top_p,
                    const float* uniforms, int dtype, int* status, void* stream) {
  if (dtype != PKV_DTYPE_F32 && dtype != PKV_DTYPE_F16 && dtype != PKV_DTYPE_BF16)
    return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  if (rows < 0 || vocab <= 0 || vocab > 0x7fffffff || row_stride < vocab)
    return fail(PKV_ERR_INVALID, "sample_rows: bad sizes rows=%lld vocab=%lld stride=%lld",
                (long long)rows, (long long)vocab, (long long)row_stride);
  if (!(temperature > 0.f) || !(temperature <= 3.402823466e38f))
    return fail(PKV_ERR_INVALID, "sample_rows: temperature must be finite and > 0");
  if (!(top_p > 0.f && top_p <= 1.f))
    return fail(PKV_ERR_INVALID, "sample_rows: top_p must be in (0, 1]");
  if (top_k < 1 || top_k > 64)
    return fail(PKV_ERR_UNSUPPORTED, "sample_rows: top_k %d outside [1, 64]", top_k);
  if (rows > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "sample_rows: %lld rows", (long long)rows);
  if (!ids || !logits || !uniforms) return fail(PKV_ERR_INVALID, "null pointer argument");
  if (((uintptr_t)logits % elem_bytes(dtype)) != 0)
    return fail(PKV_ERR_INVALID, "sample_rows: logits not aligned to the element size");
  if (rows == 0) return PKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)rows), block(kSmpThreads);
  if (dtype == PKV_DTYPE_BF16)
    hipLaunchKernelGGL((sample_rows_kernel<bf16>), grid, block, 0, s, ids,
                       static_cast<const bf16*>(logits), row_stride, (int)vocab, temperature,
                       top_k, top_p, uniforms, status);
  else if (dtype == PKV_DTYPE_F16)
    hipLaunchKernelGGL((sample_rows_kernel<f16>), grid, block, 0, s, ids,
                       static_cast<const f16*>(logits), row_stride, (int)vocab, temperature,
                       top_k, top_p, uniforms, status);
  else
    hipLaunchKernelGGL((sample_rows_kernel<float>), grid, block, 0, s, ids,
                       static_cast<const float*>(logits), row_stride, (int)vocab, temperature,
                       top_k, top_p, uniforms, status);
  return check_launch("sample_rows_kernel");
}

}  // extern "C"
