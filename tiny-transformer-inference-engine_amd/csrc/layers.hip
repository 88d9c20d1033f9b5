// The element-wise layers around the paged attention in a decoder block, as
// single kernels: RMSNorm with the residual add fused in front of it, RoPE on
// the token-major Q/K rows of a (fused) projection output, and the SwiGLU
// gate. Each replaces a chain of framework element-wise launches (cast,
// square, mean, rsqrt, multiplies; strided even/odd slices) by one pass over
// the rows, which is what a decode step at batch 128 is bound by: its rows
// are a few KB each, so launch count, not bytes, sets the time.
//
// Arithmetic follows the modules they replace:
//   RMSNorm  models/rmsnorm.py:13-17: fp32 x, mean of squares, rsqrt(+eps),
//            (x * r) * w in fp32, one rounding to the storage type. The
//            residual add before it (serving/paged_model.py:22-29) rounds
//            x + delta to the storage type first, as the framework add does.
//   RoPE     models/rope.py:21-47: cos/sin rounded to the storage type, then
//            each product and the sum/difference rounded to it, as the
//            framework's separate element-wise ops do; interleaved (even,
//            odd) pairs; no fused multiply-add, so fp32 results are bit-exact.
//   SwiGLU   kernels/fused_swiglu/kernel.py:6-19: g * sigmoid(g) * u in fp32,
//            one rounding.
#include "pkv_internal.h"

namespace pkv {
namespace {

// elements of T in one 16-byte access (V) or element-wise access (V = 2 for
// RoPE's pairs, 1 otherwise) when pointers or strides are not 16-byte aligned
template <typename T, int V>
struct Pack {
  T e[V];
};

template <typename T, int V>
__device__ __forceinline__ Pack<T, V> ld(const T* p) {
  Pack<T, V> r;
  if constexpr (V * sizeof(T) == 16) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    __builtin_memcpy(&r, &u, 16);
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) r.e[i] = p[i];
  }
  return r;
}

template <typename T, int V>
__device__ __forceinline__ void st(T* p, const Pack<T, V>& r) {
  if constexpr (V * sizeof(T) == 16) {
    uint4 u;
    __builtin_memcpy(&u, &r, 16);
    *reinterpret_cast<uint4*>(p) = u;
  } else {
#pragma unroll
    for (int i = 0; i < V; ++i) p[i] = r.e[i];
  }
}

// value rounded to the storage type and back (identity for float)
template <typename T>
__device__ __forceinline__ float rnd(float x) {
  return (float)(T)fp32_value(x);
}

struct RmsArgs {
  void* y;
  void* res_out;
  const void* x;
  const void* delta;
  const void* weight;
  int64_t x_stride;
  int64_t delta_stride;
  int dim;
  float eps;
};

constexpr int kRmsMaxWaves = 4;

// one workgroup per row; pass 1 forms the residual sum (stored) and keeps the
// row in LDS, the sum of squares is taken in the fixed order of kNormSplit
// ranges (the order the projection kernel's fused norm uses), pass 2 writes
// the output. Rows whose length is not a multiple of 32 (or above
// kNormCanonMax) use a plain strided sum instead.
template <typename T, int V>
__global__ __launch_bounds__(64 * kRmsMaxWaves) void rms_norm_kernel(RmsArgs a) {
#pragma clang fp contract(off)
  const int64_t row = blockIdx.x;
  const T* x = static_cast<const T*>(a.x) + row * a.x_stride;
  const T* h = a.delta ? static_cast<const T*>(a.delta) + row * a.delta_stride : nullptr;
  T* r = h ? static_cast<T*>(a.res_out) + row * a.dim : nullptr;
  T* y = static_cast<T*>(a.y) + row * a.dim;
  const T* w = static_cast<const T*>(a.weight);
  const int step = blockDim.x * V;
  __shared__ float xs[kNormCanonMax];
  __shared__ float gp[4 * kNormSplit];
  __shared__ float part[kRmsMaxWaves];
  const bool canon = a.dim % 32 == 0 && a.dim <= kNormCanonMax;

  float ss = 0.f;
  for (int i = threadIdx.x * V; i < a.dim; i += step) {
    Pack<T, V> xv = ld<T, V>(x + i);
    if (h) {
      const Pack<T, V> hv = ld<T, V>(h + i);
#pragma unroll
      for (int e = 0; e < V; ++e) xv.e[e] = (T)fp32_value((float)xv.e[e] + (float)hv.e[e]);
      st<T, V>(r + i, xv);
    }
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float f = (float)xv.e[e];
      if (canon) xs[i + e] = f;
      ss = ss + f * f;
    }
  }
  float tot = 0.f;
  if (canon) {
    __syncthreads();
    if (threadIdx.x < 4 * kNormSplit) {
      const int rg = threadIdx.x >> 2;  // range
      const int g = threadIdx.x & 3;    // 8-element group
      const int steps = a.dim >> 5;
      const int per = (steps + kNormSplit - 1) / kNormSplit;
      const int st1 = min((rg + 1) * per, steps);
      float acc = 0.f;
      for (int st = rg * per; st < st1; ++st)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = xs[32 * st + 8 * g + e];
          acc = acc + f * f;
        }
      gp[threadIdx.x] = acc;
    }
    __syncthreads();
#pragma unroll
    for (int rg = 0; rg < kNormSplit; ++rg)
      tot = tot + ((gp[4 * rg] + gp[4 * rg + 1]) + (gp[4 * rg + 2] + gp[4 * rg + 3]));
  } else {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    const int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) part[wv] = ss;
    __syncthreads();
    const int nw = blockDim.x >> 6;
    for (int k = 0; k < nw; ++k) tot += part[k];
  }
  const float inv = rsqrtf(tot / (float)a.dim + a.eps);

  const T* src = h ? r : x;
  for (int i = threadIdx.x * V; i < a.dim; i += step) {
    Pack<T, V> xv;
    if (canon) {
#pragma unroll
      for (int e = 0; e < V; ++e) xv.e[e] = (T)xs[i + e];
    } else {
      xv = ld<T, V>(src + i);
    }
    const Pack<T, V> wv8 = ld<T, V>(w + i);
    Pack<T, V> out;
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float n = (float)xv.e[e] * inv;
      out.e[e] = (T)fp32_value(n * (float)wv8.e[e]);
    }
    st<T, V>(y + i, out);
  }
}

struct RopeArgs {
  void* q_out;
  void* k_out;
  void* v_out;
  const void* q;
  const void* k;
  const void* v;
  int64_t q_stride;
  int64_t k_stride;
  int64_t v_stride;
  const int32_t* positions;
  const float* cos;
  const float* sin;
  int max_pos;
  int64_t n_tokens;
  int hq;
  int hkv;
  int d;
  int* status;
};

// one thread per V elements of one head row of one token; rows ordered
// [hq query heads | hkv key heads | hkv value heads (copied)]
template <typename T, int V>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
#pragma clang fp contract(off)
  const int per_row = a.d / V;
  const int rows = a.hq + a.hkv * (a.v ? 2 : 1);
  const int64_t per_tok = (int64_t)rows * per_row;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= per_tok * a.n_tokens) return;
  const int64_t t = gid / per_tok;
  const int u = (int)(gid - t * per_tok);
  const int hr = u / per_row;
  const int c = (u - hr * per_row) * V;

  const T* src;
  T* dst;
  if (hr < a.hq) {
    src = static_cast<const T*>(a.q) + t * a.q_stride + hr * a.d + c;
    dst = static_cast<T*>(a.q_out) + (t * a.hq + hr) * a.d + c;
  } else if (hr < a.hq + a.hkv) {
    const int kh = hr - a.hq;
    src = static_cast<const T*>(a.k) + t * a.k_stride + kh * a.d + c;
    dst = static_cast<T*>(a.k_out) + (t * a.hkv + kh) * a.d + c;
  } else {
    const int vh = hr - a.hq - a.hkv;
    st<T, V>(static_cast<T*>(a.v_out) + (t * a.hkv + vh) * a.d + c,
             ld<T, V>(static_cast<const T*>(a.v) + t * a.v_stride + vh * a.d + c));
    return;
  }
  int pos = a.positions[t];
  if ((unsigned)pos >= (unsigned)a.max_pos) {
    // the framework gather would fault on this index; flag it and rotate by
    // angle 0 instead of reading outside the tables
    if (a.status && u == 0) atomicOr(a.status, PKV_STATUS_BAD_POS);
    pos = 0;
  }
  const int half = a.d >> 1;
  const float* cs = a.cos + (int64_t)pos * half + (c >> 1);
  const float* sn = a.sin + (int64_t)pos * half + (c >> 1);
  const Pack<T, V> xv = ld<T, V>(src);
  Pack<T, V> out;
#pragma unroll
  for (int j = 0; j < V / 2; ++j) {
    const float cj = rnd<T>(cs[j]);
    const float sj = rnd<T>(sn[j]);
    const float xe = (float)xv.e[2 * j];
    const float xo = (float)xv.e[2 * j + 1];
    out.e[2 * j] = (T)fp32_value(rnd<T>(xe * cj) - rnd<T>(xo * sj));
    out.e[2 * j + 1] = (T)fp32_value(rnd<T>(xe * sj) + rnd<T>(xo * cj));
  }
  st<T, V>(dst, out);
}

struct SiluArgs {
  void* out;
  const void* gate;
  const void* up;
  int64_t rows;
  int64_t cols;
  int64_t gate_stride;
  int64_t up_stride;
};

template <typename T, int V>
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluArgs a) {
  const int64_t per_row = a.cols / V;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= per_row * a.rows) return;
  const int64_t r = gid / per_row;
  const int64_t c = (gid - r * per_row) * V;
  const Pack<T, V> g = ld<T, V>(static_cast<const T*>(a.gate) + r * a.gate_stride + c);
  const Pack<T, V> u = ld<T, V>(static_cast<const T*>(a.up) + r * a.up_stride + c);
  Pack<T, V> o;
#pragma unroll
  for (int e = 0; e < V; ++e) {
    o.e[e] = (T)swiglu_gate((float)g.e[e], (float)u.e[e]);
  }
  st<T, V>(static_cast<T*>(a.out) + r * a.cols + c, o);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <typename T>
int rms_launch(const RmsArgs& a, int64_t rows, bool vec, hipStream_t stream) {
  constexpr int VV = 16 / sizeof(T);
  const int V = vec ? VV : 1;
  const int nvec = (a.dim + V - 1) / V;
  int threads = ((nvec + 63) / 64) * 64;
  threads = threads < 64 ? 64 : threads > 64 * kRmsMaxWaves ? 64 * kRmsMaxWaves : threads;
  if (vec)
    hipLaunchKernelGGL((rms_norm_kernel<T, VV>), dim3((unsigned)rows), dim3(threads), 0, stream, a);
  else
    hipLaunchKernelGGL((rms_norm_kernel<T, 1>), dim3((unsigned)rows), dim3(threads), 0, stream, a);
  return check_launch("rms_norm_kernel");
}

template <typename T>
int rope_launch(const RopeArgs& a, bool vec, hipStream_t stream) {
  constexpr int VV = 16 / sizeof(T);
  const int V = vec ? VV : 2;
  const int rows = a.hq + a.hkv * (a.v ? 2 : 1);
  const int64_t total = a.n_tokens * rows * (a.d / V);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "rope: %lld threads", (long long)total);
  if (vec)
    hipLaunchKernelGGL((rope_kernel<T, VV>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((rope_kernel<T, 2>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return check_launch("rope_kernel");
}

template <typename T>
int silu_launch(const SiluArgs& a, bool vec, hipStream_t stream) {
  constexpr int VV = 16 / sizeof(T);
  const int V = vec ? VV : 1;
  const int64_t total = a.rows * (a.cols / V);
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff)
    return fail(PKV_ERR_UNSUPPORTED, "silu_mul: %lld threads", (long long)total);
  if (vec)
    hipLaunchKernelGGL((silu_mul_kernel<T, VV>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((silu_mul_kernel<T, 1>), dim3((unsigned)blocks), dim3(256), 0, stream, a);
  return check_launch("silu_mul_kernel");
}

bool known_dtype(int dtype) {
  return dtype == PKV_DTYPE_F32 || dtype == PKV_DTYPE_F16 || dtype == PKV_DTYPE_BF16;
}

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" {

int pkv_rms_norm(void* y, void* residual_out, const void* x, const void* delta,
                 const void* weight, int64_t rows, int dim, int64_t x_stride,
                 int64_t delta_stride, float eps, int dtype, void* stream) {
  if (!known_dtype(dtype)) return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  if (rows < 0 || dim <= 0) return fail(PKV_ERR_INVALID, "bad sizes rows=%lld dim=%d", (long long)rows, dim);
  if (rows > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "rms_norm: %lld rows", (long long)rows);
  if (!y || !x || !weight || (delta && !residual_out))
    return fail(PKV_ERR_INVALID, "null pointer argument");
  if (x_stride < dim || (delta && delta_stride < dim))
    return fail(PKV_ERR_INVALID, "row stride below dim");
  if (delta && residual_out == x && x_stride != dim)
    return fail(PKV_ERR_INVALID, "in-place residual needs contiguous rows (x_stride == dim)");
  if (rows == 0) return PKV_OK;
  RmsArgs a{y, delta ? residual_out : nullptr, x, delta, weight, x_stride, delta_stride, dim, eps};
  const int vv = 16 / elem_bytes(dtype);
  const bool vec = dim % vv == 0 && x_stride % vv == 0 && (!delta || delta_stride % vv == 0) &&
                   aligned16(y) && aligned16(x) && aligned16(weight) &&
                   (!delta || (aligned16(delta) && aligned16(residual_out)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PKV_DTYPE_BF16) return rms_launch<bf16>(a, rows, vec, s);
  if (dtype == PKV_DTYPE_F16) return rms_launch<f16>(a, rows, vec, s);
  return rms_launch<float>(a, rows, vec, s);
}

int pkv_rope(void* q_out, void* k_out, void* v_out, const void* q, const void* k,
             const void* v, int64_t q_stride, int64_t k_stride, int64_t v_stride,
             const int32_t* positions, const float* cos_table, const float* sin_table,
             int max_pos, int64_t n_tokens, int hq, int hkv, int d, int dtype,
             int* status, void* stream) {
  if (!known_dtype(dtype)) return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  if (n_tokens < 0 || hq < 0 || hkv < 0 || d <= 0 || (d & 1) || max_pos <= 0)
    return fail(PKV_ERR_INVALID, "bad sizes n_tokens=%lld hq=%d hkv=%d d=%d max_pos=%d",
                (long long)n_tokens, hq, hkv, d, max_pos);
  if (!positions || !cos_table || !sin_table || (hq && (!q || !q_out)) ||
      (hkv && (!k || !k_out)) || (!v) != (!v_out))
    return fail(PKV_ERR_INVALID, "null pointer argument");
  if ((hq && q_stride < (int64_t)hq * d) || (hkv && k_stride < (int64_t)hkv * d) ||
      (v && v_stride < (int64_t)hkv * d))
    return fail(PKV_ERR_INVALID, "row stride below heads * d");
  if (n_tokens == 0 || hq + hkv == 0) return PKV_OK;
  RopeArgs a{q_out, k_out, v_out, q, k, v, q_stride, k_stride, v_stride, positions, cos_table,
             sin_table, max_pos, n_tokens, hq, hkv, d, status};
  const int vv = 16 / elem_bytes(dtype);
  const bool vec = d % vv == 0 && q_stride % vv == 0 && k_stride % vv == 0 &&
                   (!v || v_stride % vv == 0) && (!hq || (aligned16(q) && aligned16(q_out))) &&
                   (!hkv || (aligned16(k) && aligned16(k_out))) &&
                   (!v || (aligned16(v) && aligned16(v_out)));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PKV_DTYPE_BF16) return rope_launch<bf16>(a, vec, s);
  if (dtype == PKV_DTYPE_F16) return rope_launch<f16>(a, vec, s);
  return rope_launch<float>(a, vec, s);
}

int pkv_silu_mul(void* out, const void* gate, const void* up, int64_t rows, int64_t cols,
                 int64_t gate_stride, int64_t up_stride, int dtype, void* stream) {
  if (!known_dtype(dtype)) return fail(PKV_ERR_INVALID, "unknown dtype %d", dtype);
  if (rows < 0 || cols <= 0) return fail(PKV_ERR_INVALID, "bad sizes rows=%lld cols=%lld",
                                         (long long)rows, (long long)cols);
  if (!out || !gate || !up) return fail(PKV_ERR_INVALID, "null pointer argument");
  if (gate_stride < cols || up_stride < cols) return fail(PKV_ERR_INVALID, "row stride below cols");
  if (rows == 0) return PKV_OK;
  SiluArgs a{out, gate, up, rows, cols, gate_stride, up_stride};
  const int vv = 16 / elem_bytes(dtype);
  const bool vec = cols % vv == 0 && gate_stride % vv == 0 && up_stride % vv == 0 &&
                   aligned16(out) && aligned16(gate) && aligned16(up);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == PKV_DTYPE_BF16) return silu_launch<bf16>(a, vec, s);
  if (dtype == PKV_DTYPE_F16) return silu_launch<f16>(a, vec, s);
  return silu_launch<float>(a, vec, s);
}

}  // extern "C"
