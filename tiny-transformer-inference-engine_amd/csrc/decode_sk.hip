// Paged MQA decode, persistent form: two 4-wavefront workgroups per CU, each
// owning an equal contiguous share of all sequences' 32-token chunks.
//
// The chunks of every (sequence, kv head) pair are laid end to end; with C
// chunks in total and W workgroups, workgroup w owns global chunks
// [R(w), R(w+1)), R(w) = floor(w C / W). Every workgroup streams the same
// amount of K/V whatever the length distribution, no workgroup is launched
// without work, and a single launch does everything:
//   - a sequence that lies entirely inside one share is finished in place
//     (its wavefronts' states are merged through LDS and written out);
//   - a sequence cut by share boundaries gets one partial (m, l, O) per
//     workgroup that touches it (its first or last segment there, so at most
//     two per workgroup); each writer releases its partial and counts itself
//     on the sequence's arrival counter, and the last to arrive merges all of
//     them and resets the counter to zero for the next launch. Nobody waits,
//     so the scheme cannot deadlock whatever the residency.
// The per-chunk pipeline is mfma_decode_common.h. Semantics are those of
// pagedattn.forward (kernels/pagedattn/pagedattn.cu:142-447) for q_len = 1.
#include "mfma_decode_common.h"

namespace pkv {
namespace {

using namespace mfma;

// 4 wavefronts per workgroup, two workgroups per CU: while one workgroup
// waits on a segment's serial latencies (table slice, Q, partial exchange),
// the other streams.
constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;

// chunks of virtual sequence v (= sequence * hkv + kv head): 0 when the
// sequence has no query this step, at least 1 otherwise (an empty context
// still owes a zero row and lse = +inf)
__device__ __forceinline__ int sk_chunks(const AttnArgs& a, int v, int& kv_len) {
  const int s = v / a.hkv;
  kv_len = 0;
  if (a.qloc) {
    const int q0 = a.qloc[s];
    const int ql = a.qloc[s + 1] - q0;
    if (ql <= 0) return 0;
    if (q0 < 0 || q0 + ql > a.n_tokens) {
      if (a.status) atomicOr(a.status, PKV_STATUS_BAD_QLOC);
      return 0;
    }
  }
  int kl = a.seq_lens[s];
  const int cap = a.max_blk << a.bs_shift;
  kl = kl < cap ? kl : cap;
  kv_len = kl > 0 ? kl : 0;
  return kv_len > 0 ? (kv_len + kChunk - 1) / kChunk : 1;
}

// first chunk of workgroup w's share, and the workgroup owning chunk x
__device__ __forceinline__ int share_start(int w, int C, int W) {
  return (int)((int64_t)w * C / W);
}
__device__ __forceinline__ int share_owner(int x, int C, int W) {
  return (int)(((int64_t)(x + 1) * W - 1) / C);
}

// Partials cross workgroups that may sit on different XCDs, whose L2s are not
// coherent with each other. They are written and read with system-scope
// relaxed accesses, which go through to memory (write-through stores,
// cache-bypassing loads) instead of relying on whole-L2 writeback /
// invalidate fences.
__device__ __forceinline__ void coherent_store2(float* p, float x, float y) {
  union { float f[2]; unsigned long long u; } b;
  b.f[0] = x;
  b.f[1] = y;
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), b.u, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void coherent_load2(const float* p, float& x, float& y) {
  union { float f[2]; unsigned long long u; } b;
  b.u = __hip_atomic_load(reinterpret_cast<unsigned long long*>(const_cast<float*>(p)),
                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  x = b.f[0];
  y = b.f[1];
}

// Partial slot that workgroup ww wrote for the sequence whose chunk 0 is
// global chunk g0, w_first being the workgroup owning g0: the sequence is
// the first segment of every contributor except possibly w_first, where it
// is the last segment unless w_first's share starts exactly at g0.
__device__ __forceinline__ int partial_slot(int ww, int w_first, int g0, int C, int W);

__device__ __forceinline__ int partial_slot(int ww, int w_first, int g0, int C, int W) {
  return 2 * ww + (ww == w_first && share_start(ww, C, W) != g0 ? 1 : 0);
}

// block-wide exclusive scan of one int per thread; returns the total
__device__ __forceinline__ int block_scan(int x, int* sh, int& excl) {
  const int t = threadIdx.x;
  sh[t] = x;
  __syncthreads();
  for (int off = 1; off < kBlock; off <<= 1) {
    const int y = t >= off ? sh[t - off] : 0;
    __syncthreads();
    sh[t] += y;
    __syncthreads();
  }
  const int incl = sh[t];
  const int total = sh[kBlock - 1];
  __syncthreads();
  excl = incl - x;
  return total;
}

template <typename T, int D, int NT, int PF, bool OFF64>
__global__ __launch_bounds__(kBlock, 2) void decode_sk_kernel(AttnArgs a, SkArgs k) {
  using Geo = ChunkGeo<D>;
  using v8 = typename Ops<T>::v8;
  constexpr int G = 16 * NT;
  constexpr int DT = D / 16;
  constexpr int WAVE_BYTES = 2 * Geo::BYTES;
  constexpr int OPITCH = D + 4;
  constexpr int MERGE_BYTES = kWaves * G * OPITCH * 4;
  constexpr int MAIN_BYTES = kWaves * WAVE_BYTES;
  constexpr int LDS_BYTES = MAIN_BYTES > MERGE_BYTES ? MAIN_BYTES : MERGE_BYTES;
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
  __shared__ float ml_lds[kWaves][G][2];
  __shared__ int tbl[kTblCap];
  __shared__ int scan_sh[kBlock];
  __shared__ int s_v0, s_off0, s_g0, s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int grp = lane >> 4;
  const int l16 = lane & 15;
  const int wg = blockIdx.x;
  const int V = a.n_seq * a.hkv;

  // ---- total chunk count C, then the sequence holding this share's start
  int C = 0;
  for (int base = 0; base < V; base += kBlock) {
    int kl;
    const int n = base + tid < V ? sk_chunks(a, base + tid, kl) : 0;
    int ex;
    C += block_scan(n, scan_sh, ex);
  }
  // at most one share per chunk, so that every share is non-empty (the
  // mergers count and read exactly the workgroups that wrote a partial)
  const int W = k.n_wg < C ? k.n_wg : C;
  if (wg >= W) return;
  const int start = share_start(wg, C, W);
  const int end = share_start(wg + 1, C, W);
  if (tid == 0) s_v0 = -1;
  __syncthreads();
  int run = 0;
  for (int base = 0; base < V; base += kBlock) {
    int kl;
    const int v = base + tid;
    const int n = v < V ? sk_chunks(a, v, kl) : 0;
    int ex;
    const int tot = block_scan(n, scan_sh, ex);
    if (n > 0 && run + ex <= start && start < run + ex + n) {
      s_v0 = v;
      s_off0 = start - (run + ex);
      s_g0 = run + ex;
    }
    run += tot;
    __syncthreads();
    if (s_v0 >= 0) break;
  }

  PoolView pv;
  pv.kbase = static_cast<const char*>(a.k_pool);
  pv.vbase = static_cast<const char*>(a.v_pool);
  pv.row_stride = (int64_t)a.hkv * D * 2;
  pv.num_blocks = (int)a.num_blocks;
  pv.bs_shift = a.bs_shift;
  ChunkCtx cx;
  cx.kl = lds + w * WAVE_BYTES;
  cx.vl = cx.kl + Geo::BYTES;
  cx.tbl = tbl;
  cx.prow = lane / Geo::CPR;
  cx.pcol = lane % Geo::CPR;
  cx.grp = grp;
  cx.l16 = l16;
  cx.scale_log2 = a.scale_log2;
  bool bad_block = false;
  const T* __restrict__ q = static_cast<const T*>(a.q);
  T* __restrict__ out = static_cast<T*>(a.out);
  float* ob = reinterpret_cast<float*>(lds);
  // kTblCap - 1 blocks of tokens: a window that starts inside a block still
  // touches at most kTblCap table entries
  const int win = (kTblCap - 1) << a.bs_shift;

  int v = s_v0;
  int c0 = s_off0;
  int g0 = s_g0;  // global index of chunk 0 of sequence v
  int remaining = end - start;
  bool first = true;
  while (remaining > 0) {
    int kv_len;
    const int n = sk_chunks(a, v, kv_len);
    if (n == 0) {
      ++v;
      continue;
    }
    const int c1 = min(n, c0 + remaining);
    const bool whole = c0 == 0 && c1 == n;
    const int s = v / a.hkv;
    const int kvh = v - s * a.hkv;
    const int64_t qrow0 = (int64_t)(a.qloc ? a.qloc[s] : s) * a.hq + kvh * G;
    const int tok_lo = c0 * kChunk;
    const int tok_hi = min(c1 * kChunk, kv_len);

    v8 qf[NT][D / 32];
    load_q<T, D, NT>(qf, q, qrow0, grp, l16);
    pv.head_off = (int64_t)kvh * D * 2;
    const int32_t* __restrict__ table = a.block_tables + (int64_t)s * a.max_blk;
    WaveState<NT, DT> st;
    st.reset();
    for (int lo = tok_lo; lo < tok_hi; lo += win) {
      cx.seg_lo = lo;
      cx.seg_hi = min(lo + win, tok_hi);
      cx.blk_lo = lo >> a.bs_shift;
      const int nblk = ((cx.seg_hi - 1) >> a.bs_shift) + 1 - cx.blk_lo;
      __syncthreads();  // previous window's table / slices no longer read
      for (int i = tid; i < nblk; i += kBlock) tbl[i] = table[cx.blk_lo + i];
      __syncthreads();
      run_chunks<T, D, NT, PF, OFF64>(w, kWaves, cx, pv, qf, st, bad_block);
    }

    // ---- merge the wavefronts' states through LDS ----
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      st.l[nt] += __shfl_xor(st.l[nt], 16);
      st.l[nt] += __shfl_xor(st.l[nt], 32);
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<floatx4*>(ob + (w * G + 16 * nt + l16) * OPITCH + 16 * dt + 4 * grp) =
            st.o[nt][dt];
    if (grp == 0) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        ml_lds[w][16 * nt + l16][0] = st.m[nt];
        ml_lds[w][16 * nt + l16][1] = st.l[nt];
      }
    }
    __syncthreads();
    const int slot = 2 * wg + (first ? 0 : 1);
    for (int idx = tid; idx < G * D / 4; idx += kBlock) {
      const int head = idx / (D / 4);
      const int d0 = (idx - head * (D / 4)) * 4;
      float M = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, ml_lds[ww][head][0]);
      float L = 0.f;
      floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
      if (M != -INFINITY) {
#pragma unroll
        for (int ww = 0; ww < kWaves; ++ww) {
          const float wt = exp2f(ml_lds[ww][head][0] - M);
          L += ml_lds[ww][head][1] * wt;
          acc += wt * *reinterpret_cast<const floatx4*>(ob + (ww * G + head) * OPITCH + d0);
        }
      }
      if (whole) {
        const int64_t qrow = qrow0 + head;
        const float inv = L > 0.f ? 1.f / L : 0.f;
        T* dst = out + qrow * D + d0;
        dst[0] = (T)(acc[0] * inv);
        dst[1] = (T)(acc[1] * inv);
        dst[2] = (T)(acc[2] * inv);
        dst[3] = (T)(acc[3] * inv);
        if (d0 == 0 && a.lse) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2f : INFINITY;
      } else {
        // written through to memory (system-coherent stores), so another
        // XCD's L2 can never hold a stale copy and no cache flush is needed
        float* po = k.part_o + ((int64_t)slot * G + head) * D + d0;
        coherent_store2(po, acc[0], acc[1]);
        coherent_store2(po + 2, acc[2], acc[3]);
        if (d0 == 0) coherent_store2(k.part_ml + ((int64_t)slot * G + head) * 2, M, L);
      }
    }

    if (!whole) {
      // every thread's write-through stores are complete before the
      // workgroup counts itself; the count and the merger's reads go to the
      // memory side too, so the last arrival sees every partial
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      const int w_first = share_owner(g0, C, W);
      const int w_last = share_owner(g0 + n - 1, C, W);
      if (tid == 0) {
        const int old = __hip_atomic_fetch_add(k.counters + v, 1, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_SYSTEM);
        s_last = old == w_last - w_first;
      }
      __syncthreads();
      if (s_last) {
        // contributors' loads are issued in unrolled batches of kMB before
        // any is consumed, so a sequence cut into many shares costs a few
        // memory latencies, not one per contributor
        constexpr int kMB = 8;
        for (int idx = tid; idx < G * D / 4; idx += kBlock) {
          const int head = idx / (D / 4);
          const int d0 = (idx - head * (D / 4)) * 4;
          float M = -INFINITY;
          for (int wb = w_first; wb <= w_last; wb += kMB) {
            float mm[kMB], ll[kMB];
#pragma unroll
            for (int i = 0; i < kMB; ++i) {
              mm[i] = -INFINITY;
              if (wb + i <= w_last)
                coherent_load2(k.part_ml + ((int64_t)partial_slot(wb + i, w_first, g0, C, W) * G +
                                            head) * 2, mm[i], ll[i]);
            }
#pragma unroll
            for (int i = 0; i < kMB; ++i) M = fmaxf(M, mm[i]);
          }
          float L = 0.f;
          floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
          if (M != -INFINITY) {
            for (int wb = w_first; wb <= w_last; wb += kMB) {
              float mm[kMB], ll[kMB], o0[kMB], o1[kMB], o2[kMB], o3[kMB];
#pragma unroll
              for (int i = 0; i < kMB; ++i) {
                mm[i] = -INFINITY;
                ll[i] = o0[i] = o1[i] = o2[i] = o3[i] = 0.f;
                if (wb + i <= w_last) {
                  const int64_t sl = partial_slot(wb + i, w_first, g0, C, W);
                  coherent_load2(k.part_ml + (sl * G + head) * 2, mm[i], ll[i]);
                  const float* po = k.part_o + (sl * G + head) * D + d0;
                  coherent_load2(po, o0[i], o1[i]);
                  coherent_load2(po + 2, o2[i], o3[i]);
                }
              }
#pragma unroll
              for (int i = 0; i < kMB; ++i) {
                const float wt = mm[i] == -INFINITY ? 0.f : exp2f(mm[i] - M);
                L += ll[i] * wt;
                acc[0] += o0[i] * wt;
                acc[1] += o1[i] * wt;
                acc[2] += o2[i] * wt;
                acc[3] += o3[i] * wt;
              }
            }
          }
          const int64_t qrow = qrow0 + head;
          const float inv = L > 0.f ? 1.f / L : 0.f;
          T* dst = out + qrow * D + d0;
          dst[0] = (T)(acc[0] * inv);
          dst[1] = (T)(acc[1] * inv);
          dst[2] = (T)(acc[2] * inv);
          dst[3] = (T)(acc[3] * inv);
          if (d0 == 0 && a.lse) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2f : INFINITY;
        }
        if (tid == 0)  // ready for the next launch
          __hip_atomic_store(k.counters + v, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      }
    }
    __syncthreads();  // LDS merge area is reused by the next segment

    remaining -= c1 - c0;
    g0 += n;
    ++v;
    c0 = 0;
    first = false;
  }
  if (bad_block && a.status) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
}

template <typename T, bool OFF64>
int launch_t(const AttnArgs& a, const SkArgs& k, hipStream_t stream) {
  const dim3 grid(k.n_wg);
  const int nt = a.group / 16;
  // <T, D, NT, PF, OFF64>: two wavefronts per SIMD (8 per CU, two workgroups)
  if (a.d == 64 && nt == 1)
    hipLaunchKernelGGL((decode_sk_kernel<T, 64, 1, 2, OFF64>), grid, dim3(kBlock), 0, stream, a, k);
  else if (a.d == 64 && nt == 2)
    hipLaunchKernelGGL((decode_sk_kernel<T, 64, 2, 2, OFF64>), grid, dim3(kBlock), 0, stream, a, k);
  else if (a.d == 128 && nt == 1)
    hipLaunchKernelGGL((decode_sk_kernel<T, 128, 1, 1, OFF64>), grid, dim3(kBlock), 0, stream, a, k);
  else if (a.d == 128 && nt == 2)
    hipLaunchKernelGGL((decode_sk_kernel<T, 128, 2, 1, OFF64>), grid, dim3(kBlock), 0, stream, a, k);
  else
    return fail(PKV_ERR_UNSUPPORTED, "decode_sk: d=%d group=%d", a.d, a.group);
  return check_launch("decode_sk_kernel");
}

}  // namespace

int launch_decode_sk(const AttnArgs& a, const SkArgs& k, int dtype, hipStream_t stream) {
  if (a.num_blocks >= (int64_t(1) << 31))
    return fail(PKV_ERR_UNSUPPORTED, "decode_sk: %lld blocks", (long long)a.num_blocks);
  const bool off64 = pool_needs_off64(a);
  if (dtype == PKV_DTYPE_BF16)
    return off64 ? launch_t<bf16, true>(a, k, stream) : launch_t<bf16, false>(a, k, stream);
  if (dtype == PKV_DTYPE_F16)
    return off64 ? launch_t<f16, true>(a, k, stream) : launch_t<f16, false>(a, k, stream);
  return fail(PKV_ERR_UNSUPPORTED, "decode_sk: dtype %d", dtype);
}

}  // namespace pkv
