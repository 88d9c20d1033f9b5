// Paged MQA decode, persistent and wavefront-specialised (gfx950): one
// workgroup per CU, each owning an equal share of all sequences' work (the
// cost line of decode_sk.hip), split between 4 producer wavefronts that
// stream and 2 or 4 consumer wavefronts that compute, so that streaming
// never stops for arithmetic or for the end of a sequence.
//
//   - The share is walked as one run of 32-token chunks (its segments, one
//     per sequence, in processing order). Producer p streams chunks p, p + 4,
//     ... straight from the pool into a ring of S LDS slots (chunk j in slot
//     j % S) with buffer_load_dwordx4 ... lds, so no registers hold data in
//     flight, and marks a slot full once its own loads have landed (vmcnt).
//     Block-table entries are scalar loads requested one chunk ahead.
//   - Every consumer reads every chunk: consumer (hg, h) computes the 16
//     query heads of head group hg (G / 16 groups) against the 16 tokens of
//     chunk half h: S^T = K Q^T with v_mfma_f32_16x16x32, the online softmax
//     (base 2, lazily moved reference, wavefront permlane reductions) and
//     O^T += V^T P^T with v_mfma_f32_16x16x16, whose operands are exactly the
//     score accumulator's layout and one transposing LDS read of V
//     (ds_read_b64_tr_b16). All consumers work on the same chunks at the same
//     time, so none runs ahead of another, and a slot goes back to its
//     producer once every consumer has counted itself out of it.
//   - At the end of a segment both halves of a head group leave their states
//     (O / l as T, fp32 (max, sum)) in the head group's LDS buffer and go on
//     at once; a consumer never does the end-of-sequence work, which would
//     hold up the ring for every wavefront. One end-worker wavefront per head
//     group takes the two states, frees the buffer, combines them (half 0
//     first) and writes the 16 heads' rows. A sequence cut by share
//     boundaries leaves one partial per share and head group (O / l as T,
//     fp32 (max, sum), written through to memory); the end worker that
//     completes the head group's arrival count merges them in contributor
//     order, as in decode_sk.hip.
//   - Within a share the segment holding its end (the head of a sequence
//     continued in the next share) is processed first, so cut sequences
//     publish their partials early and most shares end with a whole
//     sequence.
//
// Flags between wavefronts live in LDS and are polled; every wait is
// bounded (kWsSpinMax polls): a wait that runs out sets an abort flag that
// every other wait sees, all wavefronts leave, and the status word gets
// PKV_STATUS_STALLED. After the role split no workgroup barrier is used.
//
// LDS ring layout of a chunk: K rows then V rows, pitch 2D bytes, the
// 16-byte pieces of row r stored at piece index c ^ swz(r), which keeps the
// MFMA fragment reads and the transposing V^T reads free of bank conflicts
// (each LDS-DMA instruction writes 1 KiB contiguously, so padding rows is
// not possible). Semantics are those of pagedattn.forward
// (kernels/pagedattn/pagedattn.cu:142-447) for q_len = 1.
#include "mfma_decode_common.h"

namespace pkv {
namespace {

using namespace mfma;

typedef __attribute__((address_space(3))) void lds_void;

constexpr int kWsProducers = 4;
constexpr int kWsSpinMax = 1 << 22;  // polls before a wait gives up
constexpr int kWsRingBytes = 128 * 1024;
// threads of a workgroup with HG head groups: 2 HG consumers, 4 producers,
// HG end workers
constexpr int ws_block(int hg) { return 64 * (3 * hg + kWsProducers); }

template <int D>
struct WsGeo {
  static constexpr int CPR = D / 8;                 // 16-byte pieces per row
  static constexpr int ROW = 2 * D;                 // bytes per row
  static constexpr int TBYTES = kChunk * ROW;       // the K (or V) rows of a chunk
  static constexpr int CHUNK = 2 * TBYTES;          // K then V
  static constexpr int S = kWsRingBytes / CHUNK;    // ring slots
  static constexpr int R = S / kWsProducers;        // chunks in flight per producer
  static constexpr int ROWS_PER_DMA = 64 / CPR;     // rows one LDS-DMA instruction fills
  static constexpr int DMA_PER_HALF = 16 / ROWS_PER_DMA;
  static constexpr int DMA_PER_CHUNK = 4 * DMA_PER_HALF;  // K and V, two 16-row halves
  static_assert(D == 64 || D == 128, "head dim");
  static_assert(DMA_PER_CHUNK * R <= 63, "vmcnt holds a producer's loads");
  // piece slot of row r. D = 128 (16 pieces, a row spans all 64 banks):
  // 16 consecutive rows get 16 distinct slots (fragment reads), and 4
  // consecutive rows with 2 neighbouring pieces 8 distinct ones (V^T reads).
  // D = 64 (two rows per bank line): the same, counted per (row parity, slot).
  static __device__ __forceinline__ int swz(int r) {
    if constexpr (D == 128) return ((r & 7) << 1) | ((r >> 3) & 1);
    return (((r >> 1) & 3) << 1) | ((r >> 3) & 1);
  }
  static __device__ __forceinline__ int off(int r, int c) { return r * ROW + ((c ^ swz(r)) << 4); }
};

// PV product with a 16-token half: v_mfma_f32_16x16x16 (A = V^T 16 dims x 16
// tokens, B = P^T 16 tokens x 16 heads; lane l supplies row l % 16 of A and
// column l % 16 of B with the 4 k-values of group l / 16)
template <typename T>
struct Ops16;
template <>
struct Ops16<bf16> {
  typedef short v4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ floatx4 mma(v4 a, v4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};
template <>
struct Ops16<f16> {
  typedef _Float16 v4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ floatx4 mma(v4 a, v4 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};

// ---- LDS flags: accessed in inline asm, so that the wait-count pass does
// not put a vmcnt(0) (for the LDS-DMA in flight) before every access ----
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}
__device__ __forceinline__ int lds_ld(const int* p) {
  int v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(lds_addr(p)) : "memory");
  return __builtin_amdgcn_readfirstlane(v);
}
__device__ __forceinline__ void lds_st(int* p, int v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory");
}
__device__ __forceinline__ void lds_add(int* p, int v) {
  asm volatile("ds_add_u32 %0, %1" ::"v"(lds_addr(p)), "v"(v) : "memory");
}

// Flags of one workgroup.
template <int S>
struct WsFlags {
  int full[S];       // (global chunk index + 1) of the chunk whose rows have landed in the slot
  int rel[S];        // consumer releases of the slot, all uses together
  int dready[2][2];  // [head group][half]: (segment + 1) of the state deposited
  int dfree[2];      // [head group]: (segment + 1) of the deposits the end worker has taken
  int abort;         // a wait ran out: every wavefront leaves
};

// Waits until *p >= target; false (abort) when the abort flag is set or the
// poll bound runs out (then it sets the flag).
__device__ __forceinline__ bool ws_wait(const int* p, int target, int* abort_flag) {
  for (int spins = 0;; ++spins) {
    if (lds_ld(p) >= target) return true;
    if (lds_ld(abort_flag) != 0) return false;
    if (spins > kWsSpinMax) {
      lds_st(abort_flag, 1);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// One segment of a share: chunks [c0, c1) of virtual sequence v (= sequence
// * hkv + kv head), whose cost interval starts at g0 and holds n chunks.
struct WsSeg {
  int v, g0, n, kl, qtok, c0, c1;
};
__device__ __forceinline__ WsSeg ws_none() { return WsSeg{-1, 0, 0, 0, 0, 0, 0}; }

// The share's segments in processing order: the end-cut segment E first
// (when the share ends inside a sequence other than its first; the kernel
// hands it out), then the sequences from the one holding the share's start
// upward (stopping before E). Every wavefront walks the same list. Metadata
// of the next candidate is requested one step ahead (scalar loads).
struct WsWalk {
  int start, end, K, V;
  int vE;  // E's pair when E goes first, else -1
  int cand, g;
  int m_kl, m_q0, m_q1;

  struct SeqDescWs {
    int n, kv_len;
  };
  // chunks and clamped context of a pair from its query range and seq_len
  // (the rules of decode_sk.hip's seq_desc)
  static __device__ __forceinline__ SeqDescWs seq_desc_ws(const AttnArgs& a, int q0, int q1,
                                                         int kl) {
    SeqDescWs d{0, 0};
    if (a.qloc && (q1 - q0 <= 0 || q0 < 0 || q1 > a.n_tokens)) return d;
    const int cap = a.max_blk << a.bs_shift;
    kl = kl < cap ? kl : cap;
    d.kv_len = kl > 0 ? kl : 0;
    d.n = d.kv_len > 0 ? (d.kv_len + kChunk - 1) / kChunk : 1;
    return d;
  }

  __device__ __forceinline__ void request(const AttnArgs& a) {
    if (cand < V) {
      const int s = cand / a.hkv;
      m_kl = ld_meta(a.seq_lens, s);
      if (a.qloc) {
        m_q0 = ld_meta(a.qloc, s);
        m_q1 = ld_meta(a.qloc, s + 1);
      }
    }
  }
  __device__ __forceinline__ WsSeg next(const AttnArgs& a) {
    WsSeg r = ws_none();
    for (;;) {
      if (cand >= V || cand == vE) return r;
      const int s = cand / a.hkv;
      const SeqDescWs d = a.qloc ? seq_desc_ws(a, m_q0, m_q1, m_kl) : seq_desc_ws(a, 0, 1, m_kl);
      if (d.n == 0) {  // no query this step: costs nothing
        ++cand;
        request(a);
        continue;
      }
      if (g + K >= end) return r;
      r.v = cand;
      r.g0 = g;
      r.n = d.n;
      r.kl = d.kv_len;
      r.qtok = a.qloc ? m_q0 : s;
      r.c0 = max(0, start - g - K);
      r.c1 = min(d.n, end - g - K);
      if (r.c1 <= r.c0) {
        r.v = -1;
        return r;
      }
      g += d.n + K;
      ++cand;
      request(a);
      return r;
    }
  }
};

__device__ __forceinline__ int ws_share_start(int w, int C, int W) {
  return (int)((int64_t)w * C / W);
}
__device__ __forceinline__ int ws_share_owner(int x, int C, int W) {
  return (int)(((int64_t)(x + 1) * W - 1) / C);
}

// Partial slot of contributor ww of a sequence cut over [w_first, w_last]
// (decode_sk.hip's rule): its first segment's slot 2ww, except w_first's
// when its share starts with an earlier sequence (2 w_first + 1).
__device__ __forceinline__ int64_t ws_cut_slot(int ww, int w_first, int r_slot) {
  return ww == w_first ? 2 * (int64_t)ww + r_slot : 2 * (int64_t)ww;
}

__device__ __forceinline__ uint64_t ws_ld_agent64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// HG = G / 16 head groups; consumers (hg, half) = wavefronts 2hg + half.
template <typename T, int D, int HG>
struct WsKernel {
  using Geo = WsGeo<D>;
  using v8 = typename Ops<T>::v8;
  using v4 = typename Ops16<T>::v4;
  static constexpr int G = 16 * HG;
  static constexpr int DT = D / 16;
  static constexpr int KS = D / 32;
  static constexpr int S = Geo::S;
  static constexpr int R = Geo::R;
  static constexpr int NC = 2 * HG;  // consumer wavefronts
  static constexpr int BLOCK = ws_block(HG);

  struct Lds {
    char* ring;                  // [S][CHUNK]
    uint64_t (*dep)[2][DT][64];  // [HG][half]: a consumer's state, O / l as T (MFMA layout)
    float2 (*dml)[2][16];        // [HG][half]: its (max, sum) per head
    WsFlags<S>* f;
  };

  // ---------------------------------------------------------------------
  // Producer p: chunks p, p + 4, ... of the share, R in flight.
  static __device__ __forceinline__ void producer(const AttnArgs& a, WsWalk wk, WsSeg cur,
                                                  const Lds& sm, int p) {
    const int lane = threadIdx.x & 63;
    const int bs_shift = a.bs_shift;
    const int bs_mask = (1 << bs_shift) - 1;
    const int row_stride = a.hkv * D * 2;
    const unsigned nb = (unsigned)a.num_blocks;
    const char* kbase = static_cast<const char*>(a.k_pool);
    const char* vbase = static_cast<const char*>(a.v_pool);
    WsFlags<S>* f = sm.f;
    bool bad = false;
    // per lane: row within its DMA group of ROWS_PER_DMA rows, piece slot
    const int prow = lane / Geo::CPR;
    const int pslot = lane % Geo::CPR;
    int j = p;      // global index of the chunk to issue
    int jbase = 0;  // global index of cur's first chunk
    while (cur.v >= 0 && j - jbase >= cur.c1 - cur.c0) {
      jbase += cur.c1 - cur.c0;
      cur = wk.next(a);
    }
    // tokens and table entries of the chunk to issue (requested one chunk ahead)
    int e0 = 0, e1 = 0, tk0 = 0, tk1 = 0;
    auto request = [&]() {
      const int tb = (cur.c0 + j - jbase) * kChunk;
      tk0 = tb;
      tk1 = tb + 16 < cur.kl ? tb + 16 : tb;  // a half wholly past the end re-reads the first
      const int32_t* tbl = a.block_tables + (int64_t)(cur.v / a.hkv) * a.max_blk;
      e0 = ld_meta(tbl, tk0 >> bs_shift);
      e1 = ld_meta(tbl, tk1 >> bs_shift);
    };
    if (cur.v >= 0) request();
    int kc = 0;  // chunks this producer issued
    bool ok_run = true;
    while (cur.v >= 0) {
      const int slot = j % S;
      // every consumer is done with the slot's previous chunk (j - S)
      if (j >= S && !ws_wait(&f->rel[slot], NC * (j / S), &f->abort)) {
        ok_run = false;
        break;
      }
      // ---- the chunk's K and V rows into the slot ----
      {
        char* dst = sm.ring + slot * Geo::CHUNK;
        const int kvh = cur.v - (cur.v / a.hkv) * a.hkv;
        const int head_off = kvh * D * 2;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int tok = h ? tk1 : tk0;
          const int phys = h ? e1 : e0;
          const int lim = max(0, min(15, cur.kl - 1 - tok));
          const bool ok = (unsigned)phys < nb;
          bad |= !ok;
          const int64_t base =
              ((((int64_t)(ok ? phys : 0)) << bs_shift) + (tok & bs_mask)) * row_stride + head_off;
          const int extent = ok ? 16 * row_stride : 0;
          const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
              const_cast<char*>(kbase + base), (short)0, extent, kRsrcWord3);
          const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
              const_cast<char*>(vbase + base), (short)0, extent, kRsrcWord3);
#pragma unroll
          for (int i = 0; i < Geo::DMA_PER_HALF; ++i) {
            const int row = Geo::ROWS_PER_DMA * i + prow;  // row within the half
            const int rr = min(row, lim);
            const int piece = pslot ^ Geo::swz(16 * h + row);
            const unsigned voff = (unsigned)(rr * row_stride + (piece << 4));
            char* ld = dst + (16 * h + Geo::ROWS_PER_DMA * i) * Geo::ROW;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_void*)ld, 16, voff, 0, 0, 2);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_void*)(ld + Geo::TBYTES), 16, voff,
                                                     0, 0, 2);
          }
        }
      }
      // ---- this producer's next chunk, and its table entries ----
      j += kWsProducers;
      while (cur.v >= 0 && j - jbase >= cur.c1 - cur.c0) {
        jbase += cur.c1 - cur.c0;
        cur = wk.next(a);
      }
      if (cur.v >= 0) request();
      // ---- its chunk issued R - 1 before has landed once DMA_PER_CHUNK (R - 1)
      // newer loads remain ----
      if (kc >= R - 1) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(Geo::DMA_PER_CHUNK * (R - 1)) : "memory");
        const int jl = p + kWsProducers * (kc - R + 1);
        if (lane == 0) lds_st(&f->full[jl % S], jl + 1);
      }
      ++kc;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (ok_run && lane == 0)
      for (int kk = kc - R + 1 > 0 ? kc - R + 1 : 0; kk < kc; ++kk) {
        const int jl = p + kWsProducers * kk;
        lds_st(&f->full[jl % S], jl + 1);
      }
    if (bad && a.status && lane == 0) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
  }

  // ---------------------------------------------------------------------
  // Output rows (acc / L) and lse of head 16hg + l16 from the MFMA layout.
  static __device__ __forceinline__ void write_rows(const AttnArgs& a, int64_t qrow0,
                                                    const floatx4 (&acc)[DT], float M, float L,
                                                    int l16, int grp) {
    T* out = static_cast<T*>(a.out);
    const int64_t qrow = qrow0 + l16;
    const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<uint64_t*>(out + qrow * D + 16 * dt + 4 * grp) = pack4<T>(acc[dt], inv);
    if (grp == 0 && a.lse) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2f : INFINITY;
  }

  // Merge of head group hg's partials of a cut sequence by one wavefront,
  // in contributor order (the result does not depend on which contributor
  // merges); loads are device-coherent (the partials were written through
  // from other XCDs in this launch).
  static __device__ __forceinline__ void merge(const AttnArgs& a, const SkArgs& k, int hg,
                                               int w_first, int w_last, int r_slot,
                                               int64_t qrow0) {
    const int lane = threadIdx.x & 63;
    const int l16 = lane & 15, grp = lane >> 4;
    constexpr int kMB = 4;
    float M = -INFINITY, L = 0.f;
    floatx4 acc[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const uint64_t* po = reinterpret_cast<const uint64_t*>(k.part_o);
    const uint64_t* pm = reinterpret_cast<const uint64_t*>(k.part_ml);
    for (int wb = w_first; wb <= w_last; wb += kMB) {
      uint64_t mlr[kMB], oor[kMB][DT];
#pragma unroll
      for (int jj = 0; jj < kMB; ++jj) {
        const int64_t u = ws_cut_slot(min(wb + jj, w_last), w_first, r_slot) * HG + hg;
        mlr[jj] = ws_ld_agent64(pm + u * 16 + l16);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oor[jj][dt] = ws_ld_agent64(po + (u * DT + dt) * 64 + lane);
      }
#pragma unroll
      for (int jj = 0; jj < kMB; ++jj) {
        float2 ml;
        __builtin_memcpy(&ml, &mlr[jj], 8);
        if (wb + jj > w_last || ml.x == -INFINITY) continue;
        const float Mn = fmaxf(M, ml.x);
        const float sa = exp2f(M - Mn);
        const float wl = ml.y * exp2f(ml.x - Mn);
        L = L * sa + wl;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) acc[dt] = acc[dt] * sa + unpack4<T>(oor[jj][dt]) * wl;
        M = Mn;
      }
    }
    write_rows(a, qrow0, acc, M, L, l16, grp);
  }

  // ---------------------------------------------------------------------
  // Consumer (hg, half): heads 16hg ... 16hg + 15 against tokens 16half ...
  // 16half + 15 of every chunk of the share.
  static __device__ __forceinline__ void consumer(const AttnArgs& a, WsWalk wk, WsSeg cur,
                                                  const Lds& sm, int hg, int half) {
    const int lane = threadIdx.x & 63;
    const int grp = lane >> 4;
    const int l16 = lane & 15;
    const T* __restrict__ q = static_cast<const T*>(a.q);
    WsFlags<S>* f = sm.f;
    const float sc = a.scale_log2;
    auto qrow_of = [&](const WsSeg& sg) {  // first row of this head group's query heads
      const int s = sg.v / a.hkv;
      return (int64_t)sg.qtok * a.hq + (int64_t)(sg.v - s * a.hkv) * G + 16 * hg;
    };
    WsSeg nxt = cur.v >= 0 ? wk.next(a) : ws_none();
    v8 qf[1][KS], qn[1][KS];
    if (cur.v >= 0) load_q<T, D, 1>(qf, q, qrow_of(cur), grp, l16);
    if (nxt.v >= 0) load_q<T, D, 1>(qn, q, qrow_of(nxt), grp, l16);
    int j = 0;   // global index of the next chunk
    int si = 0;  // segment index
    bool aborted = false;
    while (cur.v >= 0) {
      float m = -INFINITY, l = 0.f;
      floatx4 o[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
      const int nch = cur.c1 - cur.c0;
      const int seg_hi = min(cur.c1 * kChunk, cur.kl);
      // after an aborted wait the loop still runs to the segment's end
      // (every further wait returns at once; the arithmetic on stale slots
      // is discarded), so the state has one home in registers on every path
      for (int i = 0; i < nch; ++i, ++j) {
        const int slot = j % S;
        aborted |= !ws_wait(&f->full[slot], j + 1, &f->abort);
        const char* kl = sm.ring + slot * Geo::CHUNK;
        const char* vl = kl + Geo::TBYTES;
        // the lane's fragment offsets are recomputed per chunk (a few VALU
        // instructions) rather than held across the loop in registers
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const int l16c = ln & 15, grpc = ln >> 4;
        // ---- S^T = K Q^T: tokens 16half + 4grp + r of the chunk, head l16 ----
        floatx4 sacc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const v8 kf = *reinterpret_cast<const v8*>(kl + Geo::off(16 * half + l16c, 4 * ks + grpc));
          sacc = Ops<T>::mma(kf, qf[0][ks], sacc);
        }
        // ---- online softmax (base 2): the reference m moves only when a
        // score exceeds it by more than kLazy (exact: O / l does not depend
        // on it); masked scores are -inf ----
        const int cb = (cur.c0 + i) * kChunk;
        const int lim = seg_hi - cb - 16 * half - 4 * grpc;
        float sv[4];
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sv[r] = r < lim ? sacc[r] : -INFINITY;
          mx = fmaxf(mx, sv[r]);
        }
        if (__builtin_amdgcn_ballot_w64(mx * sc > m + kLazy) != 0) {
          const float mh = head_lanes_max(mx) * sc;
          const float m_new = fmaxf(m, mh);
          const float alpha = m_new == -INFINITY ? 1.f : exp2_fast(m - m_new);
          l *= alpha;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[dt] *= alpha;
          m = m_new;
        }
        const float nref = m == -INFINITY ? 0.f : -m;
        T pt[4];
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = exp2_fast(__builtin_fmaf(sv[r], sc, nref));
          ps += pr;
          pt[r] = (T)pr;
        }
        l += ps;
        v4 pf;
        __builtin_memcpy(&pf, pt, 8);
        // ---- O^T += V^T P^T: V^T fragment (dims 16dt + l16, tokens 4grp + e
        // of the half) by one transposing read: source lane s of a 16-lane
        // group addresses row 16half + 4grp + s/4, dims 16dt + 4(s%4) ... + 3,
        // i.e. piece 2dt + (s%4)/2, byte 8(s%2) of it ----
        const int r0 = 16 * half + 4 * grpc + (l16c >> 2);
        const int sw = Geo::swz(r0);
        const char* vrow = vl + r0 * Geo::ROW + 8 * (l16c & 1);
        const int b = (l16c >> 1) & 1;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const v4s x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) v4s*)(vrow + (((2 * dt + b) ^ sw) << 4)));
          v4 vf;
          __builtin_memcpy(&vf, &x, 8);
          o[dt] = Ops16<T>::mma(vf, pf, o[dt]);
        }
        // ---- this consumer is out of the slot ----
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) lds_add(&f->rel[slot], 1);
      }
      if (aborted) break;
      // ---- end of the segment: the state goes to the end worker ----
      l = head_lanes_sum(l);
      // the end worker has taken the previous segment's deposits
      if (!ws_wait(&f->dfree[hg], si, &f->abort)) break;
      {
        const float il = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) sm.dep[hg][half][dt][lane] = pack4<T>(o[dt], il);
        if (grp == 0) sm.dml[hg][half][l16] = make_float2(m, l);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) lds_st(&f->dready[hg][half], si + 1);
      }
      // ---- next segment ----
      ++si;
      cur = nxt;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qf[0][ks] = qn[0][ks];
      nxt = cur.v >= 0 ? wk.next(a) : ws_none();
      if (nxt.v >= 0) load_q<T, D, 1>(qn, q, qrow_of(nxt), grp, l16);
    }
  }
  // ---------------------------------------------------------------------
  // End worker of head group hg: per segment, the two halves' states are
  // combined (half 0 first), then the rows or the share's partial are
  // written; the cut protocol and the merge of a completed cut sequence
  // run here, off the consumers.
  static __device__ __forceinline__ void end_worker(const AttnArgs& a, const SkArgs& k, WsWalk wk,
                                                    WsSeg cur, const Lds& sm, int hg, int C,
                                                    int W, int wg) {
    const int lane = threadIdx.x & 63;
    const int grp = lane >> 4;
    const int l16 = lane & 15;
    WsFlags<S>* f = sm.f;
    const int K = wk.K;
    int si = 0;
    while (cur.v >= 0) {
      if (!ws_wait(&f->dready[hg][0], si + 1, &f->abort)) break;
      if (!ws_wait(&f->dready[hg][1], si + 1, &f->abort)) break;
      asm volatile("" ::: "memory");
      const float2 x0 = sm.dml[hg][0][l16];
      const float2 x1 = sm.dml[hg][1][l16];
      const float M = fmaxf(x0.x, x1.x);
      const float w0 = x0.x == -INFINITY ? 0.f : x0.y * exp2f(x0.x - M);
      const float w1 = x1.x == -INFINITY ? 0.f : x1.y * exp2f(x1.x - M);
      const float L = w0 + w1;
      floatx4 o[DT];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        o[dt] = unpack4<T>(sm.dep[hg][0][dt][lane]) * w0 + unpack4<T>(sm.dep[hg][1][dt][lane]) * w1;
      // the buffer is free for the next segment's deposits
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) lds_st(&f->dfree[hg], si + 1);
      const int64_t qrow0 =
          (int64_t)cur.qtok * a.hq + (int64_t)(cur.v - (cur.v / a.hkv) * a.hkv) * G + 16 * hg;
      if (cur.c0 == 0 && cur.c1 == cur.n) {
        write_rows(a, qrow0, o, M, L, l16, grp);
      } else {
        // partial of this head group: O / L as T and (M, L), written
        // through; then count in on the head group's arrival counter
        const int w_first = ws_share_owner(cur.g0 + K, C, W);
        const int w_last = ws_share_owner(cur.g0 + K + cur.n - 1, C, W);
        const int r_slot = ws_share_start(w_first, C, W) < cur.g0 ? 1 : 0;
        const int64_t u = ws_cut_slot(wg, w_first, r_slot) * HG + hg;
        uint64_t* po = reinterpret_cast<uint64_t*>(k.part_o);
        uint64_t* pm = reinterpret_cast<uint64_t*>(k.part_ml);
        const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) st_agent64(po + (u * DT + dt) * 64 + lane, pack4<T>(o[dt], inv));
        if (grp == 0) {
          const float2 ml = make_float2(M, L);
          uint64_t bm;
          __builtin_memcpy(&bm, &ml, 8);
          st_agent64(pm + u * 16 + l16, bm);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        int cnt = 0;
        // record .w counts head group 0's contributors in, .z head group 1's
        int* ctr = reinterpret_cast<int*>(k.recs + cur.v) + 3 - hg;
        if (lane == 0) {
          cnt = fetch_add_agent(ctr, 1);
          if (cnt == w_last - w_first)
            __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if ((cnt < 0 || cnt > w_last - w_first) && a.status)
            atomicOr(a.status, PKV_STATUS_DIRTY_WORKSPACE);
        }
        cnt = __builtin_amdgcn_readlane(cnt, 0);
        if (cnt == w_last - w_first) merge(a, k, hg, w_first, w_last, r_slot, qrow0);
      }
      ++si;
      cur = wk.next(a);
    }
  }
};

template <typename T, int D, int HG>
__global__ __launch_bounds__(ws_block(HG), 1) void decode_ws_kernel(AttnArgs a, SkArgs k) {
  using WK = WsKernel<T, D, HG>;
  using Geo = WsGeo<D>;
  constexpr int S = Geo::S;
  constexpr int BLOCK = WK::BLOCK;
  constexpr int NW = BLOCK / 64;
  __shared__ __attribute__((aligned(1024))) char ring[S * Geo::CHUNK];
  __shared__ __attribute__((aligned(16))) uint64_t dep[HG][2][WK::DT][64];
  __shared__ float2 dml[HG][2][16];
  __shared__ WsFlags<S> flags;
  __shared__ int scan_sh[NW];
  __shared__ int sv[12];
  const typename WK::Lds sm{ring, dep, dml, &flags};

  const int tid = threadIdx.x;
  const int wg = blockIdx.x;
  const int V = a.n_seq * a.hkv;
  const int K = k.seg_cost;
  if (tid < S) {
    flags.full[tid] = 0;
    flags.rel[tid] = 0;
  }
  if (tid < 4) (&flags.dready[0][0])[tid] = 0;
  if (tid < 2) flags.dfree[tid] = 0;
  if (tid == 0) flags.abort = 0;
  // ---- total cost C; then the pair holding the share's start (v0) and the
  // one whose chunks hold its end (vE) ----
  const int32_t* alt = reinterpret_cast<const int32_t*>(k.recs);
  auto desc = [&](int v, int& n, int& kl, int& qtok) {
    const int s = v / a.hkv;
    const int32_t* qsrc = a.qloc ? a.qloc : alt;
    const int kv = a.seq_lens[s];
    const int q0 = qsrc[s];
    const int q1 = qsrc[a.qloc ? s + 1 : s];
    qtok = a.qloc ? q0 : s;
    const int ql = a.qloc ? q1 - q0 : 1;
    if (a.qloc && ql > 0 && (q0 < 0 || q0 + ql > a.n_tokens) && a.status && wg == 0)
      atomicOr(a.status, PKV_STATUS_BAD_QLOC);
    const WsWalk::SeqDescWs d = WsWalk::seq_desc_ws(a, a.qloc ? q0 : 0, a.qloc ? q1 : 1, kv);
    n = d.n;
    kl = d.kv_len;
  };
  // one pass when every pair fits the block (its values are kept), else a
  // second pass once C is known
  int C = 0;
  int cost_mine = 0, ex_mine = 0, n_mine = 0, kl_mine = 0, qt_mine = 0;
  for (int base = 0; base < V; base += BLOCK) {
    int n, kl, qt;
    desc(min(base + tid, V - 1), n, kl, qt);
    const int cost = base + tid < V && n > 0 ? n + K : 0;
    int ex;
    C += block_scan<NW>(cost, scan_sh, ex);
    cost_mine = cost;
    ex_mine = ex;
    n_mine = n;
    kl_mine = kl;
    qt_mine = qt;
  }
  const int W = k.n_wg < C ? k.n_wg : C;
  if (wg >= W) return;
  const int start = ws_share_start(wg, C, W);
  const int end = ws_share_start(wg + 1, C, W);
  if (tid == 0) {
    sv[0] = -1;
    sv[6] = -1;
  }
  __syncthreads();
  // v0: the pair whose cost interval holds the share's start; vE: the pair
  // whose chunks hold the share's end, short of that pair's end (an end cut)
  auto mark = [&](int v, int g, int cost, int n, int kl, int qt) {
    if (cost > 0 && g <= start && start < g + cost) {
      sv[0] = v;
      sv[1] = g;
      sv[2] = n;
      sv[3] = kl;
      sv[4] = qt;
    }
    if (cost > 0 && g + K <= end - 1 && end < g + cost) {
      sv[6] = v;
      sv[7] = g;
      sv[8] = n;
      sv[9] = kl;
      sv[10] = qt;
    }
  };
  if (V <= BLOCK) {
    mark(tid, ex_mine, cost_mine, n_mine, kl_mine, qt_mine);
  } else {
    int run = 0;
    for (int base = 0; base < V; base += BLOCK) {
      const int v = base + tid;
      int n, kl, qt;
      desc(min(v, V - 1), n, kl, qt);
      const int cost = v < V && n > 0 ? n + K : 0;
      int ex;
      const int tot = block_scan<NW>(cost, scan_sh, ex);
      mark(v, run + ex, cost, n, kl, qt);
      run += tot;
    }
  }
  __syncthreads();
  const int v0 = __builtin_amdgcn_readfirstlane(sv[0]);
  const int vE = __builtin_amdgcn_readfirstlane(sv[6]);
  const bool e_first = vE >= 0 && vE != v0;
  WsWalk wk;
  wk.start = start;
  wk.end = end;
  wk.K = K;
  wk.V = V;
  wk.vE = e_first ? vE : -1;
  wk.cand = v0 >= 0 ? v0 : V;
  wk.g = __builtin_amdgcn_readfirstlane(sv[1]);
  wk.m_kl = __builtin_amdgcn_readfirstlane(sv[3]);
  wk.m_q0 = 0;
  wk.m_q1 = 1;
  if (a.qloc && v0 >= 0) {  // the first candidate's query range
    const int s = v0 / a.hkv;
    wk.m_q0 = ld_meta(a.qloc, s);
    wk.m_q1 = ld_meta(a.qloc, s + 1);
  }
  WsSeg first;
  if (e_first) {
    first.v = vE;
    first.g0 = __builtin_amdgcn_readfirstlane(sv[7]);
    first.n = __builtin_amdgcn_readfirstlane(sv[8]);
    first.kl = __builtin_amdgcn_readfirstlane(sv[9]);
    first.qtok = __builtin_amdgcn_readfirstlane(sv[10]);
    first.c0 = 0;
    first.c1 = end - first.g0 - K;
  } else {
    first = wk.next(a);
  }
  // wavefronts: consumers [0, 2HG), producers [2HG, 2HG + 4), end workers after
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  if (w < WK::NC)
    WK::consumer(a, wk, first, sm, w >> 1, w & 1);
  else if (w < WK::NC + kWsProducers)
    WK::producer(a, wk, first, sm, w - WK::NC);
  else
    WK::end_worker(a, k, wk, first, sm, w - WK::NC - kWsProducers, C, W, wg);
  if ((tid & 63) == 0 && a.status && lds_ld(&flags.abort) != 0)
    atomicOr(a.status, PKV_STATUS_STALLED);
}

template <typename T, int D, int HG>
int launch_ws_v(const AttnArgs& a, SkArgs k, hipStream_t stream) {
  k.n_wg = ws_workgroups();
  k.seg_cost = kWsSegCost;
  hipLaunchKernelGGL((decode_ws_kernel<T, D, HG>), dim3(k.n_wg), dim3(ws_block(HG)), 0, stream, a,
                     k);
  return check_launch("decode_ws_kernel");
}

}  // namespace

int ws_workgroups() {
  const int n = device_cu_count();
  return n < kSkMaxWg ? n : kSkMaxWg;
}

bool decode_ws_supported(const AttnArgs& a, int dtype) {
  return (dtype == PKV_DTYPE_BF16 || dtype == PKV_DTYPE_F16) && !a.kv8 && a.bs_shift >= 4 &&
         a.qfilter == 0 && !a.new_pos && a.d == 128 && (a.group == 16 || a.group == 32) &&
         a.max_blk >= 1 && a.num_blocks < (int64_t(1) << 31);
}

int launch_decode_ws(const AttnArgs& a, const SkArgs& k, int dtype, hipStream_t stream) {
  if (!decode_ws_supported(a, dtype))
    return fail(PKV_ERR_UNSUPPORTED, "decode_ws: d=%d group=%d dtype %d", a.d, a.group, dtype);
  const bool bf = dtype == PKV_DTYPE_BF16;
  if (a.group == 16)
    return bf ? launch_ws_v<bf16, 128, 1>(a, k, stream) : launch_ws_v<f16, 128, 1>(a, k, stream);
  return bf ? launch_ws_v<bf16, 128, 2>(a, k, stream) : launch_ws_v<f16, 128, 2>(a, k, stream);
}

}  // namespace pkv
