// Projections of a decode step, y = x W^T (+ bias), for few rows (tokens):
// bf16/fp16 storage with fp32 accumulation on MFMA 16x16x32, or fp32
// storage on eight MFMA 16x16x4 fp32 steps per 32 k (the same lane layout),
// with the element-wise op that follows the projection in a decoder block
// fused into the epilogue:
//   plain   y rounded to the storage type            (nn.Linear)
//   swiglu  W = [gate rows; up rows]: out = g * sigmoid(g) * u of the rounded
//           gate / up outputs, rounded once  (kernels/fused_swiglu/kernel.py:6-19)
//   rope    W = [q rows; k rows; v rows] (MQA_Paged's three projections):
//           q and k rotated at positions[m], written contiguous, v copied
//           (models/rope.py:21-47 on serving/paged_mqa.py:76-85's outputs);
//           the rotation rounds exactly as the stand-alone RoPE kernel does.
//   resid   out is the residual stream, updated in place: out = out + y, y
//           rounded first and the sum rounded (PagedBlock's x + attn(...) and
//           x + mlp(...), serving/paged_model.py:20-29).
// and optionally the RMSNorm in front of the projection fused into its
// prologue (NORM): the rows are the residual stream, normalised as
// (x * rsqrt(mean(x^2) + eps)) * g in fp32 and rounded before the products
// (models/rmsnorm.py:13-17). The sum of squares is taken in one fixed order
// (each K-split wavefront's lane sums its 8-element groups step by step, the
// four groups of a row pairwise, the wavefronts in order), the order the
// stand-alone RMSNorm kernel uses too, so both give identical bits.
//
// With tokens in the tens to hundreds, a decode projection is a stream of
// the weight matrix, and the library GEMMs' large output tiles leave most of
// the chip idle with long K loops. Here a workgroup owns 16 output features
// x 16*MB rows and splits K over its 8 wavefronts (each a contiguous K
// range, so one wavefront reads 64-byte-or-longer runs of each weight row);
// the wavefronts' fp32 partials are summed through LDS in a fixed order, so
// results are deterministic and the same in every epilogue. 16-bit operands
// are loaded in whole cache lines and staged through LDS (an MFMA fragment
// is 16 rows x 64 bytes, so fragment-shaped loads request every line twice). The m tiles of
// one feature tile are dispatched to one XCD (block ids congruent mod 8), so
// their common weight rows are fetched from HBM once, into that XCD's L2.
#include "mfma_decode_common.h"

namespace pkv {
namespace {

using namespace mfma;

constexpr int kLW = kNormSplit;    // wavefronts per workgroup (K split)
constexpr int kLThreads = 64 * kLW;
constexpr int kNT = 16;            // output features per tile
constexpr int kPitch = kNT + 1;    // LDS row pitch of the partial sums (floats)
constexpr int kKB = 4;             // K steps per wavefront whose loads are in flight together

enum { kEpiPlain = 0, kEpiSwiglu = 1, kEpiRope = 2, kEpiResid = 3 };

struct LinArgs {
  void* out;          // plain / swiglu: [m, n] contiguous
  const void* x;      // [m, k], rows x_stride elements apart
  const void* w;      // [rows, k] contiguous (swiglu: 2n rows, gate then up)
  const void* bias;   // nullable, one per weight row
  int64_t x_stride;
  int m;
  int n;              // output features (swiglu: per half)
  int k;
  int m_tiles;
  int n_tiles;
  // rope epilogue
  void* q_out;
  void* k_out;
  void* v_out;
  const int32_t* positions;
  const float* cos;
  const float* sin;
  int max_pos;
  int hq;
  int hkv;
  int d;
  int* status;
  // fused RMSNorm prologue
  const void* norm_w;  // [k]
  float eps;
};

template <typename T>
__device__ __forceinline__ float rnd(float x) {
  return (float)(T)fp32_value(x);
}

// WIDE: a workgroup owns two 16-feature tiles (row sets 0 and 1 are
// features n0 .. n0 + 15 and n0 + 16 .. n0 + 31), for grids that would
// otherwise take more than one workgroup per CU (each reads its x rows for
// twice the features)
template <typename T, int MB, int EPI, bool NORM, bool WIDE>
__global__ __launch_bounds__(kLThreads) void linear_kernel(LinArgs a) {
#pragma clang fp contract(off)
  using v8 = typename Ops<T>::v8;
  constexpr int MT = 16 * MB;
  static_assert(!(WIDE && EPI == kEpiSwiglu), "SwiGLU's row sets are gate and up");
  constexpr int NS = EPI == kEpiSwiglu || WIDE ? 2 : 1;  // weight row sets
  constexpr int FT = WIDE ? 2 * kNT : kNT;               // output features per tile
  // 16-bit operands are loaded in whole 128-byte lines and staged through a
  // per-wavefront LDS region (rows of 4 K steps = 256 bytes, the 16-byte
  // chunks of row r at chunk ^ (r % 16)); an MFMA fragment load touches 16
  // rows x 64 bytes, so loading fragments straight from memory costs twice
  // the cache-line requests (each line in two instructions)
  constexpr bool STAGE = sizeof(T) == 2;
  constexpr int RWS = 16 * (NS + MB);             // staged rows: W of each set, then x
  constexpr int WAVE_STAGE = RWS * 256;           // bytes per wavefront
  constexpr int RED_BYTES = NS * MT * kPitch * 4;  // one wavefront's partial sums
  static_assert(!STAGE || RED_BYTES <= WAVE_STAGE, "partials fit the staging region");
  __shared__ float red_f[STAGE ? 1 : NS * kLW * MT * kPitch];
  __shared__ __attribute__((aligned(16))) char stage[STAGE ? kLW * WAVE_STAGE : 16];
  __shared__ float rsum[NORM ? kLW : 1][MT];
  // wavefront ww's partial sums (set s, row, column): in its staging region
  // once its operands are in registers
  auto red = [&](int s, int ww, int row, int col) -> float& {
    if constexpr (STAGE)
      return reinterpret_cast<float*>(stage + ww * WAVE_STAGE)[(s * MT + row) * kPitch + col];
    else
      return red_f[((s * kLW + ww) * MT + row) * kPitch + col];
  };

  const int b = blockIdx.x;
  const int xcd = b & 7;
  const int r = b >> 3;
  const int mt = r % a.m_tiles;
  const int nt = (r / a.m_tiles) * 8 + xcd;
  if (nt >= a.n_tiles) return;  // padding tile: the whole workgroup leaves
  const int lane = threadIdx.x & 63;
  // scalar: the K-step tests below are then scalar branches. Under a branch
  // the compiler takes as divergent it may drop the jump and rely on the
  // EXEC mask, which an MFMA instruction does not obey
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l16 = lane & 15;
  const int n0 = nt * FT;
  const int m0 = mt * MT;
  // weight row of set s for tile row r (clamped into range; the outputs of
  // clamped rows are never stored): SwiGLU's up rows follow its n gate rows
  auto wrow_of = [&](int s, int r) -> int64_t {
    if constexpr (EPI == kEpiSwiglu)
      return (int64_t)min(n0 + r, a.n - 1) + (int64_t)s * a.n;
    else
      return (int64_t)min(n0 + kNT * s + r, a.n - 1);
  };

  // operand rows
  const T* wrow[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s)
    wrow[s] = static_cast<const T*>(a.w) + wrow_of(s, l16) * a.k + (lane >> 4) * 8;
  const T* xrow[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
    xrow[mb] = static_cast<const T*>(a.x) + (int64_t)min(m0 + 16 * mb + l16, a.m - 1) * a.x_stride +
               (lane >> 4) * 8;

  // epilogue mapping: one thread per (row, feature pair); pair p of a wide
  // tile is pair p % 8 of row set p / 8
  constexpr int PPR = FT / 2;  // feature pairs per row
  static_assert(MT * PPR <= kLThreads, "one thread per pair");
  const int t = threadIdx.x;
  const int ml = t / PPR;
  const int p = t % PPR;
  const int m = m0 + ml;
  const int n = n0 + 2 * p;
  const bool live = t < MT * PPR && m < a.m && n < a.n;
  // rope: the row's position is requested before the operands
  const int qn = a.hq * a.d;
  const int kn = a.hkv * a.d;
  const bool rot = EPI == kEpiRope && live && n < qn + kn;
  int pos = 0;
  if constexpr (EPI == kEpiRope) {
    if (rot) pos = a.positions[m];
  }
  // residual: the stream's two values and the bias are requested before the
  // operands too (the epilogue would otherwise wait for them after the
  // partial sums); each (row, feature) is read and written by this thread only
  const bool two_e = n + 1 < a.n;
  float res[2] = {0.f, 0.f};
  if constexpr (EPI == kEpiResid) {
    if (live) {
      const T* o = static_cast<const T*>(a.out) + (int64_t)m * a.n + n;
      res[0] = (float)o[0];
      if (two_e) res[1] = (float)o[1];
    }
  }
  constexpr int NVB = EPI == kEpiSwiglu ? 2 : 1;  // bias sets (gate, up)
  float bia[NVB][2] = {};
  if (a.bias && live) {
    const T* bias = static_cast<const T*>(a.bias);
#pragma unroll
    for (int s = 0; s < NVB; ++s) {
      bia[s][0] = (float)bias[s * a.n + n];
      if (two_e) bia[s][1] = (float)bias[s * a.n + n + 1];
    }
  }

  // this wavefront's contiguous range of 32-wide K steps
  const int ksteps = a.k >> 5;
  const int per = (ksteps + kLW - 1) / kLW;
  const int s0 = w * per;
  const int s1 = min(s0 + per, ksteps);

  floatx4 acc[NS][MB];
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[s][mb] = floatx4{0.f, 0.f, 0.f, 0.f};
  // The wavefront's K steps in batches of kKB, every load of a batch issued
  // before the first product (indices past the range are clamped onto its
  // last step and their products skipped), so a batch costs one memory
  // round trip. Each accumulator still adds its K steps in order.
  v8 av[kKB][NS], bv[kKB][MB];
  auto load = [&](int st, v8* A, v8* B) {
#pragma unroll
    for (int s = 0; s < NS; ++s) A[s] = *reinterpret_cast<const v8*>(wrow[s] + st * 32);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) B[mb] = *reinterpret_cast<const v8*>(xrow[mb] + st * 32);
  };
  // clamp target: the range's last step (a wavefront without steps re-reads step 0)
  const int s_last = s0 < s1 ? s1 - 1 : 0;
  // staged form: load instruction (set q, j) covers rows 4j .. 4j + 3 of
  // row set q, lane -> row 4j + (lane >> 4), chunk lane & 15 = 16-byte piece
  // (chunk & 3) of K step sb + (chunk >> 2) (clamped like the direct loads)
  char* const wst = stage + w * WAVE_STAGE;
  u32x4 gl[NS + MB][4];
  auto gload = [&](int sb) {
    const int r4 = lane >> 4, ch = lane & 15;
    const int st = min(sb + (ch >> 2), s_last);
#pragma unroll
    for (int q = 0; q < NS + MB; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + r4;
        const T* src = q < NS ? static_cast<const T*>(a.w) + wrow_of(q, r) * a.k
                              : static_cast<const T*>(a.x) +
                                    (int64_t)min(m0 + 16 * (q - NS) + r, a.m - 1) * a.x_stride;
        gl[q][j] = *reinterpret_cast<const u32x4*>(src + st * 32 + (ch & 3) * 8);
      }
  };
  auto gstage = [&]() {
    const int r4 = lane >> 4, ch = lane & 15;
#pragma unroll
    for (int q = 0; q < NS + MB; ++q)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * j + r4;
        *reinterpret_cast<u32x4*>(wst + ((q * 16 + r) * 16 + (ch ^ r)) * 16) = gl[q][j];
      }
  };
  // fragments: lane -> row lane & 15, chunk 4j + (lane >> 4) for K step j
  auto gfrag = [&]() {
#pragma unroll
    for (int j = 0; j < kKB; ++j) {
      const int c = (4 * j + (lane >> 4)) ^ l16;
#pragma unroll
      for (int s = 0; s < NS; ++s)
        av[j][s] = *reinterpret_cast<const v8*>(wst + ((s * 16 + l16) * 16 + c) * 16);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
        bv[j][mb] = *reinterpret_cast<const v8*>(wst + (((NS + mb) * 16 + l16) * 16 + c) * 16);
    }
  };
  if constexpr (STAGE) {
    static_assert(kKB == 4, "a staged row holds 4 K steps");
    gload(s0);
    gstage();
    gfrag();
  } else {
#pragma unroll
    for (int j = 0; j < kKB; ++j) load(min(s0 + j, s_last), av[j], bv[j]);
  }
  if constexpr (NORM) {
    // the whole K range of this wavefront is in registers (the host keeps
    // k within kLW * kKB steps): the rows' sums of squares, then the
    // normalised operands. Lane: row 16 mb + l16, elements 32 st + 8 (lane
    // >> 4) + e of its steps st.
    const T* gw = static_cast<const T*>(a.norm_w) + (lane >> 4) * 8;
    v8 gv[kKB];
#pragma unroll
    for (int j = 0; j < kKB; ++j) gv[j] = *reinterpret_cast<const v8*>(gw + min(s0 + j, s_last) * 32);
    float inv[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < kKB; ++j) {
        if (s0 + j < s1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float f = (float)bv[j][mb][e];
            ss = ss + f * f;
          }
        }
      }
      ss = head_lanes_sum(ss);  // (g0 + g1) + (g2 + g3) over the row's 4 lane groups
      if ((lane >> 4) == 0) rsum[w][16 * mb + l16] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      float tot = 0.f;
#pragma unroll
      for (int ww = 0; ww < kLW; ++ww) tot = tot + rsum[ww][16 * mb + l16];
      inv[mb] = rsqrtf(tot / (float)a.k + a.eps);
    }
#pragma unroll
    for (int j = 0; j < kKB; ++j)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        // convert the operand again rather than keep the fp32 values of the
        // square sums alive across the barrier (64 more registers, which
        // would halve the workgroups a CU holds)
        asm volatile("" : "+v"(bv[j][mb]));
#pragma unroll
        for (int e = 0; e < 8; ++e)
          bv[j][mb][e] = (T)fp32_value(((float)bv[j][mb][e] * inv[mb]) * (float)gv[j][e]);
      }
  }
  for (int sb = s0; sb < s1; sb += kKB) {
#pragma unroll
    for (int j = 0; j < kKB; ++j) {
      if (sb + j < s1) {
#pragma unroll
        for (int s = 0; s < NS; ++s)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) acc[s][mb] = Ops<T>::mma(av[j][s], bv[j][mb], acc[s][mb]);
      }
    }
    if (sb + kKB < s1) {
      if constexpr (STAGE) {
        gload(sb + kKB);
        gstage();
        gfrag();
      } else {
#pragma unroll
        for (int j = 0; j < kKB; ++j) load(min(sb + kKB + j, s_last), av[j], bv[j]);
      }
    }
  }

  // rope: the row's table entries, requested once the products are issued
  // (the position was requested before the operands)
  float cj = 0.f, sj = 0.f;
  bool bad_pos = false;
  if constexpr (EPI == kEpiRope) {
    if (rot) {
      if ((unsigned)pos >= (unsigned)a.max_pos) {
        // the framework gather would fault on this index; flag it and
        // rotate by angle 0 instead of reading outside the tables
        bad_pos = true;
        pos = 0;
      }
      const int c = (n < qn ? n : n - qn) % a.d;
      const int64_t tix = (int64_t)pos * (a.d >> 1) + (c >> 1);
      cj = a.cos[tix];
      sj = a.sin[tix];
    }
  }

  // lane holds rows m0 + 16 mb + l16, features n0 + 4 (lane >> 4) + i
#pragma unroll
  for (int s = 0; s < NS; ++s)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) red(s, w, 16 * mb + l16, (lane >> 4) * 4 + i) = acc[s][mb][i];
  __syncthreads();

  if (!live) return;
  const bool two = n + 1 < a.n;
  constexpr int NV = EPI == kEpiSwiglu ? 2 : 1;  // value sets per thread (gate, up)
  const int se = WIDE ? p / (kNT / 2) : 0;      // the row set of a wide tile's pair
  const int pc = WIDE ? p % (kNT / 2) : p;
  float v[NV][2];
#pragma unroll
  for (int s = 0; s < NV; ++s)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float sum = 0.f;
#pragma unroll
      for (int ww = 0; ww < kLW; ++ww) sum += red(WIDE ? se : s, ww, ml, 2 * pc + j);
      v[s][j] = sum;
    }
  if (a.bias) {
#pragma unroll
    for (int s = 0; s < NV; ++s) {
      v[s][0] = fp32_value(v[s][0] + bia[s][0]);
      if (two) v[s][1] = fp32_value(v[s][1] + bia[s][1]);
    }
  }

  if constexpr (EPI == kEpiPlain) {
    T* o = static_cast<T*>(a.out) + (int64_t)m * a.n + n;
    o[0] = (T)v[0][0];
    if (two) o[1] = (T)v[0][1];
  } else if constexpr (EPI == kEpiResid) {
    T* o = static_cast<T*>(a.out) + (int64_t)m * a.n + n;
    o[0] = (T)fp32_value(res[0] + rnd<T>(v[0][0]));
    if (two) o[1] = (T)fp32_value(res[1] + rnd<T>(v[0][1]));
  } else if constexpr (EPI == kEpiSwiglu) {
    T* o = static_cast<T*>(a.out) + (int64_t)m * a.n + n;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if (j == 1 && !two) break;
      o[j] = (T)swiglu_gate(rnd<T>(v[0][j]), rnd<T>(v[1][j]));
    }
  } else {
    // n is even and every region ([q | k | v], d even) starts at an even
    // feature, so the pair (n, n + 1) is one rotation pair of one head
    const float xe = rnd<T>(v[0][0]);
    const float xo = rnd<T>(v[0][1]);
    if (!rot) {
      T* o = static_cast<T*>(a.v_out) + (int64_t)m * kn + (n - qn - kn);
      o[0] = (T)xe;
      o[1] = (T)xo;
      return;
    }
    if (bad_pos && a.status && n == 0) atomicOr(a.status, PKV_STATUS_BAD_POS);
    cj = rnd<T>(cj);
    sj = rnd<T>(sj);
    const bool isq = n < qn;
    T* o = isq ? static_cast<T*>(a.q_out) + (int64_t)m * qn + n
               : static_cast<T*>(a.k_out) + (int64_t)m * kn + (n - qn);
    o[0] = (T)fp32_value(rnd<T>(xe * cj) - rnd<T>(xo * sj));
    o[1] = (T)fp32_value(rnd<T>(xe * sj) + rnd<T>(xo * cj));
  }
}

template <typename T, int EPI, bool NORM, bool WIDE>
int launch_w(LinArgs a, int mb, hipStream_t stream) {
  constexpr int FT = WIDE ? 2 * kNT : kNT;
  a.m_tiles = (a.m + 16 * mb - 1) / (16 * mb);
  a.n_tiles = (a.n + FT - 1) / FT;
  const int64_t blocks = (int64_t)((a.n_tiles + 7) / 8) * 8 * a.m_tiles;
  if (blocks > 0x7fffffff) return fail(PKV_ERR_UNSUPPORTED, "linear: %lld tiles", (long long)blocks);
  if (mb == 1)
    hipLaunchKernelGGL((linear_kernel<T, 1, EPI, NORM, WIDE>), dim3((unsigned)blocks),
                       dim3(kLThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((linear_kernel<T, 2, EPI, NORM, WIDE>), dim3((unsigned)blocks),
                       dim3(kLThreads), 0, stream, a);
  return check_launch("linear_kernel");
}

template <typename T, int EPI, bool NORM>
int launch_t(LinArgs a, hipStream_t stream) {
  const int mb = a.m <= 16 ? 1 : 2;
  // 16-bit operands (staged through LDS: one workgroup per CU): a grid of
  // more 16-feature tiles than CUs takes two tiles per workgroup instead
  if constexpr (sizeof(T) == 2 && EPI != kEpiSwiglu) {
    const int64_t tiles = (int64_t)((a.m + 16 * mb - 1) / (16 * mb)) * ((a.n + kNT - 1) / kNT);
    if (tiles > device_cu_count()) return launch_w<T, EPI, NORM, true>(a, mb, stream);
  }
  return launch_w<T, EPI, NORM, false>(a, mb, stream);
}

template <int EPI, bool NORM = false>
int dispatch(const LinArgs& a, int dtype, hipStream_t stream) {
  if (NORM && (a.k >> 5) > kLW * kKB)
    return fail(PKV_ERR_UNSUPPORTED, "linear: fused RMSNorm needs k <= %d (got %d)",
                kLW * kKB * 32, a.k);
  if (dtype == PKV_DTYPE_BF16) return launch_t<bf16, EPI, NORM>(a, stream);
  if (dtype == PKV_DTYPE_F16) return launch_t<f16, EPI, NORM>(a, stream);
  if (dtype == PKV_DTYPE_F32) return launch_t<float, EPI, NORM>(a, stream);
  return fail(PKV_ERR_UNSUPPORTED, "linear: dtype %d", dtype);
}

int check_common(const void* out, const void* x, const void* w, int64_t m, int64_t n, int64_t k,
                 int64_t x_stride, int dtype) {
  if (dtype != PKV_DTYPE_BF16 && dtype != PKV_DTYPE_F16 && dtype != PKV_DTYPE_F32)
    return fail(PKV_ERR_UNSUPPORTED, "linear: dtype %d", dtype);
  if (m < 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x3fffffff || k > 0x7fffffff)
    return fail(PKV_ERR_INVALID, "linear: bad sizes m=%lld n=%lld k=%lld", (long long)m,
                (long long)n, (long long)k);
  if (!out || !x || !w) return fail(PKV_ERR_INVALID, "linear: null pointer argument");
  if (k % 32 != 0 || x_stride % 8 != 0 || ((uintptr_t)x & 15) || ((uintptr_t)w & 15))
    return fail(PKV_ERR_UNSUPPORTED,
                "linear: k (%lld) must be a multiple of 32, x rows 16-byte aligned",
                (long long)k);
  if (x_stride < k) return fail(PKV_ERR_INVALID, "linear: x_stride below k");
  return PKV_OK;
}

}  // namespace
}  // namespace pkv

namespace pkv {
namespace {
// q/k/v projection with RoPE, optionally with the RMSNorm fused in front
// (norm_weight non-null)
int rope_qkv(void* q_out, void* k_out, void* v_out, const void* x, const void* norm_weight,
             float eps, const void* w_qkv, const void* bias, int64_t m, int64_t k,
             int64_t x_stride, const int32_t* positions, const float* cos_table,
             const float* sin_table, int max_pos, int hq, int hkv, int d, int dtype, int* status,
             void* stream) {
  if (hq <= 0 || hkv <= 0 || d <= 0 || (d & 1) || max_pos <= 0)
    return fail(PKV_ERR_INVALID, "linear_rope_qkv: bad sizes hq=%d hkv=%d d=%d max_pos=%d", hq,
                hkv, d, max_pos);
  const int64_t n = (int64_t)(hq + 2 * hkv) * d;
  const int rc = check_common(q_out, x, w_qkv, m, n, k, x_stride, dtype);
  if (rc != PKV_OK) return rc;
  if (!k_out || !v_out || !positions || !cos_table || !sin_table)
    return fail(PKV_ERR_INVALID, "linear_rope_qkv: null pointer argument");
  if (m == 0) return PKV_OK;
  LinArgs a{};
  a.x = x;
  a.w = w_qkv;
  a.bias = bias;
  a.x_stride = x_stride;
  a.m = (int)m;
  a.n = (int)n;
  a.k = (int)k;
  a.q_out = q_out;
  a.k_out = k_out;
  a.v_out = v_out;
  a.positions = positions;
  a.cos = cos_table;
  a.sin = sin_table;
  a.max_pos = max_pos;
  a.hq = hq;
  a.hkv = hkv;
  a.d = d;
  a.status = status;
  a.norm_w = norm_weight;
  a.eps = eps;
  if (norm_weight) return dispatch<kEpiRope, true>(a, dtype, static_cast<hipStream_t>(stream));
  return dispatch<kEpiRope>(a, dtype, static_cast<hipStream_t>(stream));
}
}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" {

int pkv_linear(void* out, const void* x, const void* w, const void* bias, int64_t m, int64_t n,
               int64_t k, int64_t x_stride, int dtype, void* stream) {
  const int rc = check_common(out, x, w, m, n, k, x_stride, dtype);
  if (rc != PKV_OK || m == 0) return rc;
  LinArgs a{};
  a.out = out;
  a.x = x;
  a.w = w;
  a.bias = bias;
  a.x_stride = x_stride;
  a.m = (int)m;
  a.n = (int)n;
  a.k = (int)k;
  return dispatch<kEpiPlain>(a, dtype, static_cast<hipStream_t>(stream));
}

int pkv_linear_swiglu(void* out, const void* x, const void* w_gate_up, const void* bias,
                      int64_t m, int64_t n, int64_t k, int64_t x_stride, int dtype,
                      void* stream) {
  const int rc = check_common(out, x, w_gate_up, m, n, k, x_stride, dtype);
  if (rc != PKV_OK || m == 0) return rc;
  LinArgs a{};
  a.out = out;
  a.x = x;
  a.w = w_gate_up;
  a.bias = bias;
  a.x_stride = x_stride;
  a.m = (int)m;
  a.n = (int)n;
  a.k = (int)k;
  return dispatch<kEpiSwiglu>(a, dtype, static_cast<hipStream_t>(stream));
}

int pkv_linear_residual(void* resid, const void* x, const void* w, const void* bias, int64_t m,
                        int64_t n, int64_t k, int64_t x_stride, int dtype, void* stream) {
  const int rc = check_common(resid, x, w, m, n, k, x_stride, dtype);
  if (rc != PKV_OK || m == 0) return rc;
  LinArgs a{};
  a.out = resid;
  a.x = x;
  a.w = w;
  a.bias = bias;
  a.x_stride = x_stride;
  a.m = (int)m;
  a.n = (int)n;
  a.k = (int)k;
  return dispatch<kEpiResid>(a, dtype, static_cast<hipStream_t>(stream));
}

int pkv_linear_swiglu_rmsnorm(void* out, const void* x, const void* norm_weight, float eps,
                              const void* w_gate_up, const void* bias, int64_t m, int64_t n,
                              int64_t k, int64_t x_stride, int dtype, void* stream) {
  int rc = check_common(out, x, w_gate_up, m, n, k, x_stride, dtype);
  if (rc != PKV_OK) return rc;
  if (!norm_weight || ((uintptr_t)norm_weight & 15))
    return fail(PKV_ERR_INVALID, "linear_swiglu_rmsnorm: norm weight null or not 16-byte aligned");
  if (m == 0) return PKV_OK;
  LinArgs a{};
  a.out = out;
  a.x = x;
  a.w = w_gate_up;
  a.bias = bias;
  a.x_stride = x_stride;
  a.m = (int)m;
  a.n = (int)n;
  a.k = (int)k;
  a.norm_w = norm_weight;
  a.eps = eps;
  return dispatch<kEpiSwiglu, true>(a, dtype, static_cast<hipStream_t>(stream));
}

int pkv_linear_rope_qkv_rmsnorm(void* q_out, void* k_out, void* v_out, const void* x,
                                const void* norm_weight, float eps, const void* w_qkv,
                                const void* bias, int64_t m, int64_t k, int64_t x_stride,
                                const int32_t* positions, const float* cos_table,
                                const float* sin_table, int max_pos, int hq, int hkv, int d,
                                int dtype, int* status, void* stream) {
  if (!norm_weight || ((uintptr_t)norm_weight & 15))
    return fail(PKV_ERR_INVALID, "linear_rope_qkv_rmsnorm: norm weight null or not 16-byte aligned");
  return rope_qkv(q_out, k_out, v_out, x, norm_weight, eps, w_qkv, bias, m, k, x_stride, positions,
                  cos_table, sin_table, max_pos, hq, hkv, d, dtype, status, stream);
}

int pkv_linear_rope_qkv(void* q_out, void* k_out, void* v_out, const void* x, const void* w_qkv,
                        const void* bias, int64_t m, int64_t k, int64_t x_stride,
                        const int32_t* positions, const float* cos_table,
                        const float* sin_table, int max_pos, int hq, int hkv, int d, int dtype,
                        int* status, void* stream) {
  return rope_qkv(q_out, k_out, v_out, x, nullptr, 0.f, w_qkv, bias, m, k, x_stride, positions,
                  cos_table, sin_table, max_pos, hq, hkv, d, dtype, status, stream);
}

}  // extern "C"


