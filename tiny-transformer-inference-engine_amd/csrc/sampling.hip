// Token selection after the vocabulary projection: greedy (argmax) and the
// scheduler's temperature / top-k / top-p draw.
//
// Greedy: the index of the largest logit of every row (serving/generation.py
// takes logits.argmax per sequence; the reference's sampler,
// sampling.py:5-137, is greedy = argmax). Same result as the framework's
// argmax: the first index holding the maximum, and a NaN counts as larger
// than every number (the first NaN wins).
//
// Argmax has two launch shapes:
//  - one workgroup per row (no workspace, or many rows);
//  - split rows: P workgroups per row, each over a slice of the vocabulary,
//    so a batch of 128 rows fills the 256 CUs and every thread has one
//    round of loads. The slices meet through the caller's workspace: each
//    folds its best into the row's key word, counts itself in on the row's
//    arrival counter (agent-scope atomics), and the slice that brings the
//    count to P writes the index and puts both words back to zero for the
//    next call. No workgroup waits for another.
// Sampling uses one workgroup per row (a split form measured slower: the
// slices' hand-over and merge cost more than the shorter passes saved);
// 16-bit rows of up to 65536 entries are held in registers between its
// steps (sample_rows_reg_kernel).
#include <algorithm>
#include <climits>
#include <type_traits>

#include "pkv_internal.h"

namespace pkv {
namespace {

__device__ __forceinline__ uint64_t xchg_agent64(uint64_t* p, uint64_t v) {
  return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t fetch_max_agent64(uint64_t* p, uint64_t v) {
  return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// From this many rows on, one workgroup per row already fills the device.
constexpr int64_t kSplitRowsMax = 512;
// Spacing of the per-row counters and key words: one cache line each.
constexpr int kLineBytes = 128;
constexpr int kCtrStride = kLineBytes / 4;
constexpr int kKeyStride = kLineBytes / 8;

// ---------------------------------------------------------------- argmax
//
// A workgroup streams its range of the row with 16-byte loads (a scalar head
// up to the first 16-byte boundary, since rows of an odd vocabulary start
// unaligned, then vectors, then a scalar tail), keeping per thread the
// largest argmax key (make_key: the framework's order as one unsigned
// comparison); the keys are combined across the wavefront by lane swaps and
// across wavefronts through LDS.
//
// 16-bit logits take a packed pass: per 32-bit word of two elements, the
// two value keys with v_pk_* operations, each joined with the element's
// position among the thread's elements of the round into a signed 32-bit
// key (value key above, 31 - position below), and a 3-way maximum; once per
// round the winner becomes a 64-bit key with its row index. About 4 VALU
// instructions per element instead of 12. A round holding a NaN (its
// magnitude bits above those of infinity) is redone with exact per-element
// keys from the registers it was loaded into.

constexpr int kAmThreads = 512;    // one workgroup per row
constexpr int kAsThreads = 256;    // split rows
constexpr int kAmUnroll = 8;      // 16-byte loads in flight per thread
constexpr int kNanKey = 0x7fffffff;

// Value key: the two's complement of the sign-magnitude bits (so the order
// is that of the numbers and -0, +0 share key 0); every NaN kNanKey, above
// every number.
template <typename T>
__device__ __forceinline__ int value_key(T v) {
  if constexpr (sizeof(T) == 2) {
    unsigned short b;
    __builtin_memcpy(&b, &v, 2);
    constexpr unsigned kInf = std::is_same<T, bf16>::value ? 0x7f80u : 0x7c00u;
    const unsigned m = b & 0x7fffu;
    if (m > kInf) return kNanKey;
    return (b & 0x8000u) ? -(int)m : (int)m;
  } else {
    const unsigned u = __float_as_uint(v);
    const unsigned m = u & 0x7fffffffu;
    if (m > 0x7f800000u) return kNanKey;
    return (u & 0x80000000u) ? -(int)m : (int)m;
  }
}

// 64-bit key whose unsigned order is argmax order: the value key (offset to
// unsigned), then the complemented index (a lower index is larger). 0 is
// below every key of an element.
__device__ __forceinline__ uint64_t make_key(int vkey, int i) {
  return ((uint64_t)((unsigned)vkey ^ 0x80000000u) << 32) | (uint64_t)(~(unsigned)i);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// The largest argmax key among vectors [v_lo, v_hi) of a row (16-byte
// vectors after the scalar head of `head` elements), plus the head when
// `with_head` and the scalar tail when `with_tail`, over NT threads. The
// loads of a round are unconditional (indices past the range clamped onto
// its last vector) so that all of them are in flight together: a load under
// a branch gets a wait of its own. A clamped copy of the last vector is
// never the workgroup's winner: the thread that loads that vector at its
// own position holds the same values at a lower index.
template <typename T, int NT>
__device__ __forceinline__ uint64_t argmax_scan(const T* __restrict__ row, int vocab, int head,
                                                int v_lo, int v_hi, bool with_head,
                                                bool with_tail, int tid) {
  constexpr int V = 16 / sizeof(T);
  uint64_t best = 0;
  if (with_head && tid < head) best = make_key(value_key(row[tid]), tid);
  const T* vrow = row + head;
  for (int it0 = v_lo; it0 < v_hi; it0 += NT * kAmUnroll) {
    const int v0 = it0 + tid;
    uint4 raw[kAmUnroll];
#pragma unroll
    for (int u = 0; u < kAmUnroll; ++u)
      raw[u] = *reinterpret_cast<const uint4*>(vrow + (int64_t)min(v0 + u * NT, v_hi - 1) * V);
    bool exact = true;
    if constexpr (sizeof(T) == 2) {
      constexpr unsigned kInf = std::is_same<T, bf16>::value ? 0x7f80u : 0x7c00u;
      constexpr int kLast = kAmUnroll * V - 1;  // the round's last position (an inline constant)
      int b32 = INT_MIN;
      u16x2 mag = {0, 0};
#pragma unroll
      for (int u = 0; u < kAmUnroll; ++u) {
        const unsigned w4[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const unsigned m = w4[w] & 0x7fff7fffu;
          const s16x2 neg = __builtin_bit_cast(s16x2, w4[w]) >> (s16x2){15, 15};
          const s16x2 key = (__builtin_bit_cast(s16x2, m) ^ neg) - neg;
          mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2, m));
          const unsigned kp = __builtin_bit_cast(unsigned, key);
          const int pos = u * V + 2 * w;  // position of element (u, 2w) in the round
          const int klo = (int)((kp << 16) | (unsigned)(kLast - pos));
          const int khi = (int)((kp & 0xffff0000u) | (unsigned)(kLast - 1 - pos));
          b32 = max(b32, max(klo, khi));
        }
      }
      exact = max((unsigned)mag.x, (unsigned)mag.y) > kInf;
      if (!exact) {
        const int pos = kLast - (b32 & 0xffff);
        best = max_u64(best, make_key(b32 >> 16, head + (v0 + (pos / V) * NT) * V + pos % V));
      }
    }
    if (exact) {
#pragma unroll
      for (int u = 0; u < kAmUnroll; ++u) {
        const int vv = v0 + u * NT;
        T e[V];
        __builtin_memcpy(e, &raw[u], 16);
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const uint64_t k = make_key(value_key(e[j]), head + vv * V + j);
          best = vv < v_hi ? max_u64(best, k) : best;
        }
      }
    }
  }
  if (with_tail) {
    const int nvec = (vocab - head) / V;
    for (int ix = head + nvec * V + tid; ix < vocab; ix += NT)
      best = max_u64(best, make_key(value_key(row[ix]), ix));
  }
  return best;
}

template <int S>
__device__ __forceinline__ uint64_t lane_xor64(uint64_t v) {
  const unsigned lo = __float_as_uint(lane_xor<S>(__uint_as_float((unsigned)v)));
  const unsigned hi = __float_as_uint(lane_xor<S>(__uint_as_float((unsigned)(v >> 32))));
  return ((uint64_t)hi << 32) | lo;
}

// The workgroup's largest key; valid in thread 0.
template <int NT>
__device__ __forceinline__ uint64_t argmax_reduce(uint64_t best, int tid) {
  best = max_u64(best, lane_xor64<1>(best));
  best = max_u64(best, lane_xor64<2>(best));
  best = max_u64(best, lane_xor64<4>(best));
  best = max_u64(best, lane_xor64<8>(best));
  best = max_u64(best, lane_xor64<16>(best));
  best = max_u64(best, lane_xor64<32>(best));
  __shared__ uint64_t s_k[NT / 64];
  if ((tid & 63) == 0) s_k[tid >> 6] = best;
  __syncthreads();
  if (tid == 0)
    for (int w = 1; w < NT / 64; ++w) best = max_u64(best, s_k[w]);
  return best;
}

__device__ __forceinline__ int row_head(const void* row, int vocab, int esize) {
  return min(vocab, (int)(((16 - ((uintptr_t)row & 15)) & 15) / esize));
}

template <typename T>
__global__ __launch_bounds__(kAmThreads) void argmax_rows_kernel(int64_t* __restrict__ ids,
                                                                 const T* __restrict__ logits,
                                                                 int64_t row_stride, int vocab) {
  constexpr int V = 16 / sizeof(T);
  const T* row = logits + (int64_t)blockIdx.x * row_stride;
  const int tid = threadIdx.x;
  const int head = row_head(row, vocab, sizeof(T));
  uint64_t best = argmax_scan<T, kAmThreads>(row, vocab, head, 0, (vocab - head) / V, true, true, tid);
  best = argmax_reduce<kAmThreads>(best, tid);
  if (tid == 0) ids[blockIdx.x] = (int64_t)(~(unsigned)(best & 0xffffffffu));
}

// Split rows: workgroup (slice, row) scans vectors [slice * per, ...) of the
// row (slice 0 also the head, the last slice the tail) and folds its best
// into the row's key word with an agent-scope atomic max; then it counts
// itself in. The last of the row's slices reads the key (exchanging it for
// 0) and writes the index. Every key is in the word before its slice's
// increment: the max returns before the add is issued (both are performed at
// the memory side, where every XCD meets).
template <typename T>
__global__ __launch_bounds__(kAsThreads) void argmax_split_kernel(
    int64_t* __restrict__ ids, const T* __restrict__ logits, int64_t row_stride, int vocab,
    int nsplit, int* __restrict__ ctr, uint64_t* __restrict__ keys) {
  constexpr int V = 16 / sizeof(T);
  const int r = blockIdx.y;
  const int sl = blockIdx.x;
  const T* row = logits + (int64_t)r * row_stride;
  const int tid = threadIdx.x;
  const int head = row_head(row, vocab, sizeof(T));
  const int nvec = (vocab - head) / V;
  const int per = (nvec + nsplit - 1) / nsplit;
  const int v_lo = min(nvec, sl * per);
  const int v_hi = min(nvec, v_lo + per);
  uint64_t best = argmax_scan<T, kAsThreads>(row, vocab, head, v_lo, v_hi, sl == 0,
                                             sl == nsplit - 1, tid);
  best = argmax_reduce<kAsThreads>(best, tid);
  if (tid == 0) {
    // an empty slice folds key 0: below every element's key
    uint64_t* kw = keys + (int64_t)r * kKeyStride;
    int* cw = ctr + (int64_t)r * kCtrStride;
    fetch_max_agent64(kw, best);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const int old = fetch_add_agent(cw, 1);
    if (old == nsplit - 1) {
      const uint64_t k = xchg_agent64(kw, 0);
      __hip_atomic_store(cw, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ids[r] = (int64_t)(~(unsigned)(k & 0xffffffffu));
    }
  }
}

// ------------------------------------------------- top-k / top-p sampling
//
// sampling.py:5-137's sample(): temperature, apply_top_k, apply_top_p,
// softmax, one multinomial draw; the reference's top-k kernel,
// kernels/cuda-kSAMPLING/ksampling_kernel.cu:61-185, covers the top-k step
// alone. Per row (one workgroup, or each slice of a split row):
//   1. y = x / temperature (fp32, correctly rounded), the range's
//      finiteness, and each thread's maximum;
//   2. t0 = the k-th largest of the 256 thread maxima (each wavefront sorts
//      its 64 across the lanes, and the four lists are merged with lane
//      shuffles): at least k values of the range are >= t0, so every value
//      of the range's top-k set is;
//   3. the values >= t0 (normally k to a few k of them) are collected in
//      LDS and sorted descending (ties by ascending index; a rank sort up to
//      256 of them): the k-th is the range's top-k threshold, and its
//      survivors (every value >= it, ties kept, as apply_top_k's
//      `logits < kth` mask keeps them) are a prefix;
//   4. one wavefront takes the softmax over the row's survivors, the
//      cumulative mass in that order, keeps the prefix whose mass before
//      each token is at most top_p (the first always), renormalises, and
//      picks the token by inverse CDF in vocabulary order: the first kept
//      index (ascending) whose cumulative probability exceeds u * total, u
//      the row's uniform.
// More than kSmpCand values >= t0 in a row (only with massive ties) sets
// PKV_STATUS_SAMPLE_OVERFLOW and writes -1: the caller samples that call
// another way. A non-finite logit
// sets PKV_STATUS_NONFINITE, a non-finite scaled value (temperature
// underflow) PKV_STATUS_BAD_DISTRIBUTION.
constexpr int kSmpThreads = 256;
constexpr int kSmpCand = 1024;
constexpr int kSmpUnroll = 8;      // 16-byte loads in flight per thread

// Candidates are packed into one 64-bit key whose unsigned order is the
// sort order (larger value first, then smaller index): the value's bits made
// monotone (-0 as +0; the values are finite or -inf) above the complemented
// index.
__device__ __forceinline__ uint64_t smp_pack(float v, int i) {
  const unsigned u = v == 0.f ? 0u : __float_as_uint(v);
  const unsigned hi = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)hi << 32) | (uint64_t)(~(unsigned)i);
}
__device__ __forceinline__ float smp_value(uint64_t k) {
  const unsigned hi = (unsigned)(k >> 32);
  return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7fffffffu) : ~hi);
}
__device__ __forceinline__ int smp_index(uint64_t k) { return (int)~(unsigned)(k & 0xffffffffu); }

// Descending bitonic sort of n (a power of two <= kSmpCand) LDS keys, for
// candidate sets too large for the rank sort. Pair p of a stage joins
// i = 2p - (p & (stride - 1)) and i + stride; thread t takes pairs t,
// t + 256, ...: for strides up to 64 every element wavefront w touches lies
// in its own blocks [128 (w + 4m), + 128), so those stages need no
// workgroup barrier (a wavefront's LDS accesses complete in order), only
// the stages with longer strides and the ones right after them.
template <int NT>
__device__ __forceinline__ void smp_bitonic(uint64_t* key, int n) {
  __syncthreads();
  int prev_stride = 0;
  for (int size = 2; size <= n; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= 128 || prev_stride >= 128)
        __syncthreads();
      else
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      prev_stride = stride;
      for (int p = threadIdx.x; p < (n >> 1); p += NT) {
        const int i = 2 * p - (p & (stride - 1));
        const int j = i + stride;
        const uint64_t ki = key[i], kj = key[j];
        const bool swap = (i & size) == 0 ? kj > ki : ki > kj;
        if (swap) {
          key[i] = kj;
          key[j] = ki;
        }
      }
    }
  }
  __syncthreads();
}

// Sorts the n keys ck descending. Up to kSmpThreads keys: each thread ranks
// its key by counting the larger ones (every lane reads the same entry at a
// time: broadcast LDS reads, no branches) and writes it to sk[rank]; the
// result is in sk. More: bitonic sort in place, result in ck.
template <int NT>
__device__ __forceinline__ uint64_t* smp_sort(uint64_t* ck, uint64_t* sk, int n) {
  const int tid = threadIdx.x;
  __syncthreads();
  if (n <= kSmpThreads) {
    if (tid < n) {
      const uint64_t me = ck[tid];
      int r = 0;
#pragma unroll 8
      for (int j = 0; j < n; ++j) r += ck[j] > me ? 1 : 0;
      sk[r] = me;
    }
    __syncthreads();
    return sk;
  }
  int m = 64;
  while (m < n) m <<= 1;
  for (int i = n + tid; i < m; i += NT) ck[i] = 0;  // below every key
  smp_bitonic<NT>(ck, m);
  return ck;
}

// Inclusive prefix sum across the wavefront's lanes: DPP row shifts within
// each row of 16 lanes, then the totals of the earlier rows (read lanes).
__device__ __forceinline__ float wave_incl_scan(float x) {
  const int lane = threadIdx.x & 63;
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xF, 0xF, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xF, 0xF, false));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 15));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 31));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 47));
  const int rw = lane >> 4;
  const float before = rw == 0 ? 0.f : (rw == 1 ? r0 : (rw == 2 ? r0 + r1 : (r0 + r1) + r2));
  return x + before;
}

__device__ __forceinline__ int wave_min_i(int x) {
  x = min(x, __float_as_int(lane_xor<32>(__int_as_float(x))));
  x = min(x, __float_as_int(lane_xor<16>(__int_as_float(x))));
  x = min(x, __float_as_int(lane_xor<8>(__int_as_float(x))));
  x = min(x, __float_as_int(lane_xor<4>(__int_as_float(x))));
  x = min(x, __float_as_int(lane_xor<2>(__int_as_float(x))));
  return min(x, __float_as_int(lane_xor<1>(__int_as_float(x))));
}
__device__ __forceinline__ int wave_max_i(int x) {
  x = max(x, __float_as_int(lane_xor<32>(__int_as_float(x))));
  x = max(x, __float_as_int(lane_xor<16>(__int_as_float(x))));
  x = max(x, __float_as_int(lane_xor<8>(__int_as_float(x))));
  x = max(x, __float_as_int(lane_xor<4>(__int_as_float(x))));
  x = max(x, __float_as_int(lane_xor<2>(__int_as_float(x))));
  return max(x, __float_as_int(lane_xor<1>(__int_as_float(x))));
}

__device__ __forceinline__ float smp_wave_sum(float x) {
  x += lane_xor<32>(x);
  x += lane_xor<16>(x);
  x += lane_xor<8>(x);
  x += lane_xor<4>(x);
  x += lane_xor<2>(x);
  return x + lane_xor<1>(x);
}

// One compare-exchange step of a descending bitonic network at distance S
// within blocks of SIZE lanes.
template <int SIZE, int S>
__device__ __forceinline__ float bitonic_step(float v) {
  const int lane = threadIdx.x & 63;
  const float o = lane_xor<S>(v);
  // descending blocks keep the larger value at the lower lane
  const bool keep_max = ((lane & SIZE) == 0) == ((lane & S) == 0);
  return keep_max ? fmaxf(v, o) : fminf(v, o);
}

// The wavefront's 64 lane values sorted descending across the lanes (lane
// i holds the i-th largest): a bitonic sort with lane shuffles.
__device__ __forceinline__ float wave_sort_desc(float v) {
  v = bitonic_step<2, 1>(v);
  v = bitonic_step<4, 2>(v);
  v = bitonic_step<4, 1>(v);
  v = bitonic_step<8, 4>(v);
  v = bitonic_step<8, 2>(v);
  v = bitonic_step<8, 1>(v);
  v = bitonic_step<16, 8>(v);
  v = bitonic_step<16, 4>(v);
  v = bitonic_step<16, 2>(v);
  v = bitonic_step<16, 1>(v);
  v = bitonic_step<32, 16>(v);
  v = bitonic_step<32, 8>(v);
  v = bitonic_step<32, 4>(v);
  v = bitonic_step<32, 2>(v);
  v = bitonic_step<32, 1>(v);
  v = bitonic_step<64, 32>(v);
  v = bitonic_step<64, 16>(v);
  v = bitonic_step<64, 8>(v);
  v = bitonic_step<64, 4>(v);
  v = bitonic_step<64, 2>(v);
  return bitonic_step<64, 1>(v);
}

// b[63 - lane]: lane ^ 63, as six exchanges
__device__ __forceinline__ float lane_reverse(float b) {
  b = lane_xor<32>(b);
  b = lane_xor<16>(b);
  b = lane_xor<8>(b);
  b = lane_xor<4>(b);
  b = lane_xor<2>(b);
  return lane_xor<1>(b);
}

// The top 64 of two descending 64-lists a, b (lane i holds a[i], b[i]),
// descending: max(a[i], b[63 - i]) is a bitonic sequence holding them, which
// half-cleaners sort.
__device__ __forceinline__ float wave_merge_top(float a, float b) {
  float v = fmaxf(a, lane_reverse(b));
  v = bitonic_step<64, 32>(v);
  v = bitonic_step<64, 16>(v);
  v = bitonic_step<64, 8>(v);
  v = bitonic_step<64, 4>(v);
  v = bitonic_step<64, 2>(v);
  return bitonic_step<64, 1>(v);
}

// The k-th largest (1 <= k <= 64) of the workgroup's 256 thread values:
// each wavefront sorts its 64 and stages them in LDS (wt: [4][64]); every
// wavefront then merges the four lists itself (no second barrier).
__device__ __forceinline__ float block_kth_largest(float v, int k, float* wt) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  wt[tid] = wave_sort_desc(v);
  __syncthreads();
  const float x = wave_merge_top(wt[lane], wt[64 + lane]);
  const float y = wave_merge_top(wt[128 + lane], wt[192 + lane]);
  const float top = wave_merge_top(x, y);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(top), k - 1));
}

struct SmpRange {
  int lo, hi;  // elements [lo, hi) of the row
};

// Calls f(x, index) for every element of the range, each thread taking its
// share: a scalar head up to the first 16-byte boundary, then 16-byte
// vectors (kSmpUnroll of them in flight per thread, loaded unconditionally:
// indices past the range are clamped onto its last vector and their
// elements skipped), then a scalar tail.
template <typename T, typename F>
__device__ __forceinline__ void smp_visit(const T* __restrict__ row, SmpRange rg, int tid, F&& f) {
  constexpr int V = 16 / sizeof(T);
  const T* base = row + rg.lo;
  const int len = rg.hi - rg.lo;
  const int head = min(len, (int)(((16 - ((uintptr_t)base & 15)) & 15) / sizeof(T)));
  if (tid < head) f((float)base[tid], rg.lo + tid);
  const int nvec = (len - head) / V;
  const T* vb = base + head;
  for (int v0 = tid; v0 < nvec; v0 += kSmpThreads * kSmpUnroll) {
    uint4 raw[kSmpUnroll];
#pragma unroll
    for (int u = 0; u < kSmpUnroll; ++u)
      raw[u] = *reinterpret_cast<const uint4*>(vb + (int64_t)min(v0 + u * kSmpThreads, nvec - 1) * V);
#pragma unroll
    for (int u = 0; u < kSmpUnroll; ++u) {
      const int vv = v0 + u * kSmpThreads;
      T e[V];
      __builtin_memcpy(e, &raw[u], 16);
      if (vv < nvec) {
#pragma unroll
        for (int j = 0; j < V; ++j) f((float)e[j], rg.lo + head + vv * V + j);
      }
    }
  }
  for (int ix = head + nvec * V + tid; ix < len; ix += kSmpThreads) f((float)base[ix], rg.lo + ix);
}

// Step 1 over the range: the thread's maximum of y and the status bits
// (temperature 1 divides exactly by skipping the division).
template <typename T, bool UNIT>
__device__ __forceinline__ void smp_pass1(const T* __restrict__ row, SmpRange rg,
                                          float temperature, int tid, float& mx, int& flags) {
  smp_visit(row, rg, tid, [&](float x, int) {
    const float y = UNIT ? x : x / temperature;
    flags |= !isfinite(x) ? PKV_STATUS_NONFINITE : 0;
    flags |= (isfinite(x) && !isfinite(y)) ? PKV_STATUS_BAD_DISTRIBUTION : 0;
    mx = fmaxf(mx, y);
  });
}

// Step 3's collection: the range's values >= t0 appended to ck as packed
// keys (cnt counts every one, also past kSmpCand). Per batch of vectors a
// thread first sets a bit per element >= t0 (branch-free), then appends the
// rare hits.
template <typename T, bool UNIT>
__device__ __forceinline__ void smp_collect(const T* __restrict__ row, SmpRange rg,
                                            float temperature, float t0, int tid, uint64_t* ck,
                                            int* cnt) {
  constexpr int V = 16 / sizeof(T);
  constexpr int HW = (V * kSmpUnroll + 63) / 64;  // hit words per batch
  auto append = [&](float y, int ix) {
    const int at = atomicAdd(cnt, 1);
    if (at < kSmpCand) ck[at] = smp_pack(y, ix);
  };
  auto scale = [&](float x) { return UNIT ? x : x / temperature; };
  const T* base = row + rg.lo;
  const int len = rg.hi - rg.lo;
  const int head = min(len, (int)(((16 - ((uintptr_t)base & 15)) & 15) / sizeof(T)));
  if (tid < head) {
    const float y = scale((float)base[tid]);
    if (y >= t0) append(y, rg.lo + tid);
  }
  const int nvec = (len - head) / V;
  const T* vb = base + head;
  for (int v0 = tid; v0 < nvec; v0 += kSmpThreads * kSmpUnroll) {
    uint4 raw[kSmpUnroll];
#pragma unroll
    for (int u = 0; u < kSmpUnroll; ++u)
      raw[u] = *reinterpret_cast<const uint4*>(vb + (int64_t)min(v0 + u * kSmpThreads, nvec - 1) * V);
    uint64_t hit[HW];
#pragma unroll
    for (int w = 0; w < HW; ++w) hit[w] = 0;
#pragma unroll
    for (int u = 0; u < kSmpUnroll; ++u) {
      T e[V];
      __builtin_memcpy(e, &raw[u], 16);
      const bool ok = v0 + u * kSmpThreads < nvec;
#pragma unroll
      for (int j = 0; j < V; ++j) {
        const int b = u * V + j;
        hit[b / 64] |= (ok && scale((float)e[j]) >= t0) ? 1ull << (b % 64) : 0ull;
      }
    }
#pragma unroll
    for (int w = 0; w < HW; ++w) {
      while (hit[w]) {  // rare: the few values >= t0
        const int b = 64 * w + __builtin_ctzll(hit[w]);
        hit[w] &= hit[w] - 1;
        const int ix = head + (v0 + (b / V) * kSmpThreads) * V + b % V;
        append(scale((float)base[ix]), rg.lo + ix);
      }
    }
  }
  for (int ix = head + nvec * V + tid; ix < len; ix += kSmpThreads) {
    const float y = scale((float)base[ix]);
    if (y >= t0) append(y, rg.lo + ix);
  }
}

// LDS of the sampling kernels
struct SmpLds {
  uint64_t* ck;  // [kSmpCand] candidate keys
  uint64_t* sk;  // [kSmpThreads] rank-sorted keys
  float* qv;     // [kSmpCand] kept probabilities (step 4)
  float* wt;     // [kSmpThreads] the wavefronts' sorted thread maxima
  int* cnt;
  int* flags;
};

// Steps 1-3 over one range. Returns the status bits of the range (flags, or
// PKV_STATUS_SAMPLE_OVERFLOW); on 0, *sorted holds the nc candidates sorted.
// t0 is the k-th largest thread maximum: k threads hold a value >= t0, so
// the range's top-k set lies at or above it.
template <typename T>
__device__ __forceinline__ int smp_candidates(const T* __restrict__ row, SmpRange rg,
                                              float temperature, int k, int tid, SmpLds L,
                                              uint64_t*& sorted, int& nc) {
  if (tid == 0) {
    *L.cnt = 0;
    *L.flags = 0;
  }
  float mx = -INFINITY;
  int flags = 0;
  const bool unit_temp = temperature == 1.f;
  if (unit_temp)
    smp_pass1<T, true>(row, rg, temperature, tid, mx, flags);
  else
    smp_pass1<T, false>(row, rg, temperature, tid, mx, flags);
  if (flags) atomicOr(L.flags, flags);
  const float t0 = block_kth_largest(mx, k, L.wt);
  __syncthreads();
  const int fl = *L.flags;
  if (fl) return fl;
  if (unit_temp)
    smp_collect<T, true>(row, rg, temperature, t0, tid, L.ck, L.cnt);
  else
    smp_collect<T, false>(row, rg, temperature, t0, tid, L.ck, L.cnt);
  __syncthreads();
  nc = *L.cnt;
  if (nc > kSmpCand) return PKV_STATUS_SAMPLE_OVERFLOW;
  sorted = smp_sort<kSmpThreads>(L.ck, L.sk, nc);
  return 0;
}

// Step 4 (wavefront 0 only, lane = threadIdx.x): sk sorted, nc valid keys,
// every value of the row's top-k set among them. Lane l takes sorted
// positions l, l + 64, ...
__device__ __forceinline__ void smp_draw(const uint64_t* sk, float* qv, int nc, int k,
                                         float top_p, float u, int64_t* out, int lane) {
  const uint64_t tkey = sk[k - 1] & 0xffffffff00000000ull;  // the k-th value's bits
  // survivors: the sorted prefix >= the k-th value (ties kept)
  int ns = 0;
  for (int b = 0; b < nc; b += 64) {
    const int p = b + lane;
    ns += __popcll(__ballot(p < nc && sk[p] >= tkey));
  }
  const float m = smp_value(sk[0]);
  float zl = 0.f;
  for (int b = 0; b < ns; b += 64) {
    const int p = b + lane;
    zl += p < ns ? expf(smp_value(sk[p]) - m) : 0.f;
  }
  const float z = smp_wave_sum(zl);
  // top-p: keep a position while the mass before it (sorted order) is at
  // most top_p; the first always. Masses before a position only grow, so
  // the kept positions are a prefix.
  int nk = 0;
  float carry = 0.f;
  for (int b = 0; b < ns; b += 64) {
    const int p = b + lane;
    const float pv = p < ns ? expf(smp_value(sk[p]) - m) / z : 0.f;
    const float incl = wave_incl_scan(pv);
    const float before = carry + (incl - pv);
    nk += __popcll(__ballot(p < ns && (p == 0 || before <= top_p)));
    carry += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(incl), 63));
  }
  // renormalised probabilities of the kept prefix
  float zk_l = 0.f;
  for (int b = 0; b < nk; b += 64) {
    const int p = b + lane;
    zk_l += p < nk ? expf(smp_value(sk[p]) - m) : 0.f;
  }
  const float zk = smp_wave_sum(zk_l);
  float tot_l = 0.f;
  for (int b = 0; b < nk; b += 64) {
    const int p = b + lane;
    const float q = p < nk ? expf(smp_value(sk[p]) - m) / zk : 0.f;
    tot_l += q;
    if (p < nk) qv[p] = q;
  }
  const float target = u * smp_wave_sum(tot_l);
  __builtin_amdgcn_wave_barrier();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  // inverse CDF in vocabulary order: token i's cumulative start is the sum
  // of the kept probabilities of smaller indices (in sorted order)
  int pick = 0x7fffffff, last = -1;
  for (int b = 0; b < nk; b += 64) {
    const int p = b + lane;
    const int my = p < nk ? smp_index(sk[p]) : 0x7fffffff;
    float c = 0.f;
#pragma unroll 8
    for (int j = 0; j < nk; ++j) c += smp_index(sk[j]) < my ? qv[j] : 0.f;
    if (p < nk) {
      if (c + qv[p] > target) pick = min(pick, my);
      last = max(last, my);
    }
  }
  pick = wave_min_i(pick);
  last = wave_max_i(last);
  if (lane == 0) *out = pick != 0x7fffffff ? pick : last;
}

#define SMP_LDS_DECL                                                   \
  __shared__ uint64_t smp_ck[kSmpCand];                                \
  __shared__ uint64_t smp_sk[kSmpThreads];                             \
  __shared__ float smp_qv[kSmpCand];                                   \
  __shared__ float smp_wt[kSmpThreads];                                \
  __shared__ int smp_cnt, smp_flags;                                   \
  const SmpLds L{smp_ck, smp_sk, smp_qv, smp_wt, &smp_cnt, &smp_flags};

template <typename T>
__global__ __launch_bounds__(kSmpThreads) void sample_rows_kernel(
    int64_t* __restrict__ ids, const T* __restrict__ logits, int64_t row_stride, int vocab,
    float temperature, int top_k, float top_p, const float* __restrict__ uniforms,
    int* __restrict__ status) {
  SMP_LDS_DECL
  const int tid = threadIdx.x;
  const T* row = logits + (int64_t)blockIdx.x * row_stride;
  const int k = top_k < vocab ? top_k : vocab;
  int nc = 0;
  uint64_t* sorted = nullptr;
  const int fl = smp_candidates<T>(row, SmpRange{0, vocab}, temperature, k, tid, L, sorted, nc);
  if (fl) {
    if (tid == 0) {
      ids[blockIdx.x] = -1;
      if (status) atomicOr(status, fl);
    }
    return;
  }
  if (tid >= 64) return;
  smp_draw(sorted, L.qv, nc, k, top_p, uniforms[blockIdx.x], ids + blockIdx.x, tid);
}

// ------------------------------------------ sampling, rows held in registers
//
// 16-bit logits whose row fits one round of loads of a 512-thread workgroup
// (R 16-byte vectors per thread): the row is read once and kept in
// registers as value keys (value_key's order, computed two at a time with
// v_pk_* operations in place of the loaded words), so step 3 reads no
// memory. Same steps and results as sample_rows_kernel:
//   1. per thread: the largest key and the largest magnitude (finiteness);
//      the thread maximum of y is the value of that key divided by the
//      temperature (division by a positive number is monotone);
//   2. t0 = the k-th largest of the 512 thread maxima (wavefront 0 merges
//      the eight sorted lists);
//   3. kx = the smallest key whose scaled value is >= t0 (t0's own key at
//      temperature 1, else a binary search over the keys); per vector the
//      packed saturating differences key - kx are ANDed, and only vectors
//      with a key >= kx are walked element by element and appended;
//   4. the sort and the draw.
// Clamped copies of the row's last vector (loads past the row) count for
// neither the maxima nor the candidates.
constexpr int kSrThreads = 512;

// The 16-bit value of a key (the inverse of value_key for numbers).
template <typename T>
__device__ __forceinline__ float key16_value(int key) {
  const unsigned short b =
      key >= 0 ? (unsigned short)key : (unsigned short)(0x8000u | (unsigned)(-key));
  T v;
  __builtin_memcpy(&v, &b, 2);
  return (float)v;
}

// The k-th largest (1 <= k <= 64) of the 512 thread values: each wavefront
// sorts its 64 into wt, wavefront 0 merges the eight lists and leaves the
// result in *out. Ends with a barrier.
__device__ __forceinline__ void block_kth_largest512(float v, int k, float* wt, float* out) {
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  wt[tid] = wave_sort_desc(v);
  __syncthreads();
  if (tid < 64) {
    const float a = wave_merge_top(wt[lane], wt[64 + lane]);
    const float b = wave_merge_top(wt[128 + lane], wt[192 + lane]);
    const float c = wave_merge_top(wt[256 + lane], wt[320 + lane]);
    const float d = wave_merge_top(wt[384 + lane], wt[448 + lane]);
    const float top = wave_merge_top(wave_merge_top(a, b), wave_merge_top(c, d));
    // read with every lane active: inside a one-lane branch the compiler may
    // leave lane k - 1's value of `top` uncomputed
    const float kth = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(top), k - 1));
    if (lane == 0) *out = kth;
  }
  __syncthreads();
}

template <typename T, int R>
__global__ __launch_bounds__(kSrThreads) void sample_rows_reg_kernel(
    int64_t* __restrict__ ids, const T* __restrict__ logits, int64_t row_stride, int vocab,
    float temperature, int top_k, float top_p, const float* __restrict__ uniforms,
    int* __restrict__ status) {
  constexpr int V = 8;
  constexpr int NT = kSrThreads;
  constexpr unsigned kInf = std::is_same<T, bf16>::value ? 0x7f80u : 0x7c00u;
  __shared__ uint64_t smp_ck[kSmpCand];
  __shared__ uint64_t smp_sk[kSmpThreads];
  __shared__ float smp_qv[kSmpCand];
  __shared__ float smp_wt[kSrThreads];
  __shared__ int smp_cnt, smp_flags;
  __shared__ float smp_t0;
  const int tid = threadIdx.x;
  const T* row = logits + (int64_t)blockIdx.x * row_stride;
  const int k = top_k < vocab ? top_k : vocab;
  const bool unit = temperature == 1.f;
  const int head = row_head(row, vocab, 2);
  const int nvec = (vocab - head) / V;  // >= 1: the host sends rows of 16 elements or more
  const int tail0 = head + nvec * V;
  if (tid == 0) {
    smp_cnt = 0;
    smp_flags = 0;
  }
  uint4 kv[R];
#pragma unroll
  for (int u = 0; u < R; ++u)
    kv[u] = *reinterpret_cast<const uint4*>(row + head + (int64_t)min(tid + u * NT, nvec - 1) * V);
  // the thread's scalar element, if any: threads 0-7 the head, 8-15 the tail
  const int xi = tid < head ? tid : (tid >= 8 && tid - 8 < vocab - tail0 ? tail0 + tid - 8 : -1);
  int xk = INT_MIN;
  unsigned xm = 0;
  if (xi >= 0) {
    unsigned short b;
    __builtin_memcpy(&b, &row[xi], 2);
    xm = b & 0x7fffu;
    xk = (b & 0x8000u) ? -(int)xm : (int)xm;
  }
  // 1. keys in place, the thread's largest key and magnitude
  s16x2 best = {-32768, -32768};
  u16x2 mag = {0, 0};
#pragma unroll
  for (int u = 0; u < R; ++u) {
    unsigned w4[4] = {kv[u].x, kv[u].y, kv[u].z, kv[u].w};
    s16x2 vb = {-32768, -32768};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const unsigned m = w4[w] & 0x7fff7fffu;
      const s16x2 neg = __builtin_bit_cast(s16x2, w4[w]) >> (s16x2){15, 15};
      const s16x2 key = (__builtin_bit_cast(s16x2, m) ^ neg) - neg;
      mag = __builtin_elementwise_max(mag, __builtin_bit_cast(u16x2, m));
      vb = __builtin_elementwise_max(vb, key);
      w4[w] = __builtin_bit_cast(unsigned, key);
    }
    kv[u] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    if (tid + u * NT < nvec) best = __builtin_elementwise_max(best, vb);
  }
  const int tkey = max(max((int)best.x, (int)best.y), xk);
  const unsigned tmag = max(max((unsigned)mag.x, (unsigned)mag.y), xm);
  int flags = tmag >= kInf ? PKV_STATUS_NONFINITE : 0;
  if (!unit) {
    // a finite value whose scaled value is not finite: test the largest
    // finite magnitude (with a non-finite value present, found element by
    // element)
    unsigned fm = tmag;
    if (tmag >= kInf) {
      fm = xm < kInf ? xm : 0;
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const unsigned w4[4] = {kv[u].x, kv[u].y, kv[u].z, kv[u].w};
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int key = (int)(short)(w4[w] >> (16 * h));
            const unsigned m = (unsigned)abs(key);
            fm = m < kInf ? max(fm, m) : fm;
          }
      }
    }
    if (!isfinite(key16_value<T>((int)fm) / temperature)) flags |= PKV_STATUS_BAD_DISTRIBUTION;
  }
  float mx = -INFINITY;
  if (tkey > -32768) {  // the thread holds an element
    const float v = key16_value<T>(tkey);
    mx = unit ? v : v / temperature;
  }
  // 2. t0 (the barriers inside also order the counters' set-up before use)
  block_kth_largest512(mx, k, smp_wt, &smp_t0);
  if (flags) atomicOr(&smp_flags, flags);
  __syncthreads();
  const int fl = smp_flags;
  if (fl) {
    if (tid == 0) {
      ids[blockIdx.x] = -1;
      if (status) atomicOr(status, fl);
    }
    return;
  }
  const float t0 = smp_t0;
  // 3. the key threshold, then the candidates
  int kx = -(int)kInf;
  if (t0 > -INFINITY) {
    if (unit) {
      const T tv = (T)t0;
      unsigned short b;
      __builtin_memcpy(&b, &tv, 2);
      kx = (b & 0x8000u) ? -(int)(b & 0x7fffu) : (int)(b & 0x7fffu);
    } else {
      // smallest key with key16_value(key) / temperature >= t0: the scaled
      // value is monotone in the key, +inf's key qualifies, -inf's does not
      int lo = -(int)kInf, hi = (int)kInf;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (key16_value<T>(mid) / temperature >= t0)
          hi = mid;
        else
          lo = mid;
      }
      kx = hi;
    }
  }
  const s16x2 kxv = {(short)kx, (short)kx};
  auto append = [&](int key, int ix) {
    const float v = key16_value<T>(key);
    const float y = unit ? v : v / temperature;
    const int at = atomicAdd(&smp_cnt, 1);
    if (at < kSmpCand) smp_ck[at] = smp_pack(y, ix);
  };
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const unsigned w4[4] = {kv[u].x, kv[u].y, kv[u].z, kv[u].w};
    unsigned acc = 0xffffffffu;
#pragma unroll
    for (int w = 0; w < 4; ++w)
      acc &= __builtin_bit_cast(unsigned,
                                __builtin_elementwise_sub_sat(__builtin_bit_cast(s16x2, w4[w]), kxv));
    const int vv = tid + u * NT;
    if ((acc & 0x80008000u) != 0x80008000u && vv < nvec) {  // rare: a key >= kx
#pragma unroll
      for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int key = (int)(short)(w4[w] >> (16 * h));
          if (key >= kx) append(key, head + vv * V + 2 * w + h);
        }
    }
  }
  if (xi >= 0 && xk >= kx) append(xk, xi);
  __syncthreads();
  const int nc = smp_cnt;
  if (nc > kSmpCand) {
    if (tid == 0) {
      ids[blockIdx.x] = -1;
      if (status) atomicOr(status, PKV_STATUS_SAMPLE_OVERFLOW);
    }
    return;
  }
  const uint64_t* sorted = smp_sort<kSrThreads>(smp_ck, smp_sk, nc);
  if (tid >= 64) return;
  smp_draw(sorted, smp_qv, nc, k, top_p, uniforms[blockIdx.x], ids + blockIdx.x, tid);
}

// ------------------------------------------------------------- host side

// Workspace of the split argmax: [rows] arrival counters and [rows] key
// words, each on a 128-byte line of its own (atomics on one line are
// performed one after another at the memory side).
size_t ws_ctr_bytes(int64_t rows) { return (size_t)rows * kLineBytes; }
size_t ws_key_bytes(int64_t rows) { return (size_t)rows * kLineBytes; }

int argmax_splits(int64_t rows, int64_t vocab, int dtype) {
  if (rows >= kSplitRowsMax) return 1;
  const int64_t per = (int64_t)kAsThreads * kAmUnroll * (16 / elem_bytes(dtype));
  return (int)std::min<int64_t>(64, std::max<int64_t>(1, (vocab + per - 1) / per));
}
size_t argmax_ws_bytes(int64_t rows) { return ws_ctr_bytes(rows) + ws_key_bytes(rows); }

}  // namespace
}  // namespace pkv

using namespace pkv;

extern "C" {

size_t pkv_argmax_workspace_bytes(int64_t rows, int64_t vocab, int dtype) {
  if (rows <= 0 || vocab <= 0 || argmax_splits(rows, vocab, dtype) == 1) return 0;
  return argmax_ws_bytes(rows);
}

int pkv_argmax_rows(int64_t* ids, const void* logits, int64_t rows, int64_t vocab,
                    int64_t row_stride, int dtype, void* workspace, size_t workspace_bytes,
                    void* stream) {
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
  const int nsplit = argmax_splits(rows, vocab, dtype);
  if (nsplit > 1 && workspace && workspace_bytes >= argmax_ws_bytes(rows)) {
    if (((uintptr_t)workspace & 255) != 0)
      return fail(PKV_ERR_WORKSPACE, "argmax_rows: workspace not 256-byte aligned");
    int* ctr = static_cast<int*>(workspace);
    uint64_t* keys = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + ws_ctr_bytes(rows));
    const dim3 grid((unsigned)nsplit, (unsigned)rows), block(kAsThreads);
    if (dtype == PKV_DTYPE_BF16)
      hipLaunchKernelGGL((argmax_split_kernel<bf16>), grid, block, 0, s, ids,
                         static_cast<const bf16*>(logits), row_stride, (int)vocab, nsplit, ctr, keys);
    else if (dtype == PKV_DTYPE_F16)
      hipLaunchKernelGGL((argmax_split_kernel<f16>), grid, block, 0, s, ids,
                         static_cast<const f16*>(logits), row_stride, (int)vocab, nsplit, ctr, keys);
    else
      hipLaunchKernelGGL((argmax_split_kernel<float>), grid, block, 0, s, ids,
                         static_cast<const float*>(logits), row_stride, (int)vocab, nsplit, ctr,
                         keys);
    return check_launch("argmax_split_kernel");
  }
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
  const int64_t nvec_max = (vocab + 7) / 8;  // 16-byte vectors of a 16-bit row, at most
  if (dtype != PKV_DTYPE_F32 && vocab >= 16 && nvec_max <= kSrThreads * 16) {
    const dim3 grid((unsigned)rows), block(kSrThreads);
    const bool r8 = nvec_max <= kSrThreads * 8;
#define SR_LAUNCH(TT, RR)                                                                     \
  hipLaunchKernelGGL((sample_rows_reg_kernel<TT, RR>), grid, block, 0, s, ids,                \
                     static_cast<const TT*>(logits), row_stride, (int)vocab, temperature, top_k, \
                     top_p, uniforms, status)
    if (dtype == PKV_DTYPE_BF16) {
      if (r8) SR_LAUNCH(bf16, 8); else SR_LAUNCH(bf16, 16);
    } else {
      if (r8) SR_LAUNCH(f16, 8); else SR_LAUNCH(f16, 16);
    }
#undef SR_LAUNCH
    return check_launch("sample_rows_reg_kernel");
  }
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
