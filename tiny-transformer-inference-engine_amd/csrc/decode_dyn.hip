// Paged MQA decode, dynamic persistent form: one 8-wavefront workgroup per
// CU takes work items from a list ordered largest first.
//
// Work items. Every (sequence, kv head) pair v with a query has n_v 32-token
// chunks. A pair with more than P chunks is cut into ceil(n_v / P) equal
// pieces (a "long" pair); every other pair is one whole item. The list puts
// all pieces first (they are the largest items), then the whole items by
// size class (floor(log2 n_v), largest first), each group in pair order.
// Every workgroup builds the same list in LDS from seq_lens (and
// query_start_loc) at the start: a block scan over the piece counts and
// per-class ranks from wavefront ballots, so the order is deterministic.
//
// Schedule. With W workgroups, workgroup w takes items w and 2W - 1 - w
// (largest with smallest of the next W), then draws further items from an
// atomic counter, one item ahead, so a workgroup that streams faster (a
// less loaded XCD, shorter items) simply takes more, and the items left for
// the end are the smallest: the launch ends within about one small item of
// its ideal balance. Every workgroup draws until a draw comes back empty,
// exactly once, so the draw that brings the counter to its final count
// knows no other draw follows and resets it to zero for the next call.
//
// Pieces. A piece leaves a partial (m, l, O/l) in the slot of its item
// index. Its workgroup then adds one to the pair's arrival counter; the one
// that brings it to the number of pieces merges every partial, writes the
// output row and resets the counter. Partials and counters go through
// device-scope (agent) coherent accesses: on gfx950 those stores write
// through the XCD's L2 and those loads bypass it, so a workgroup on one XCD
// sees what another wrote once the counter says so, with no cache-wide
// writeback or invalidate. A piece's arrival is signalled at the end of its
// workgroup's next item (its partial stores have completed by then), so it
// costs no wait; pieces come first, so their merges happen while the rest
// of the list streams. No workgroup waits for another: no deadlock whatever
// the residency.
//
// Items stream through the chunk pipeline of mfma_decode_common.h, dealt
// round-robin to the 8 wavefronts; their states are merged through LDS at
// the item's end, while the next item's Q and first table window load.
// Semantics are those of pagedattn.forward
// (kernels/pagedattn/pagedattn.cu:142-447) for q_len = 1.
#include "mfma_decode_common.h"

namespace pkv {
namespace {

using namespace mfma;

constexpr int kWaves = 8;
constexpr int kBlock = 64 * kWaves;
constexpr int kClasses = 16;  // size classes of whole items
static_assert(kDynMaxSeq <= 2 * kBlock, "the list build handles two pairs per thread");
static_assert(kDynMaxSeq * 2 <= kDynItemCap, "pieces need room besides the whole items");
static_assert((kDynMaxSeq + 1) * sizeof(int) <= kWsDynCtrBytes, "counters fit their header");

// chunks of pair v this call: 0 when its sequence has no query (or another
// launch of a split batch takes it), at least 1 otherwise (an empty context
// still owes a zero row and lse = +inf)
__device__ __forceinline__ int dyn_chunks(const AttnArgs& a, int v, int& kv_len) {
  const int s = v / a.hkv;
  kv_len = 0;
  if (a.qloc) {
    const int q0 = a.qloc[s];
    const int ql = a.qloc[s + 1] - q0;
    if (ql <= 0 || (a.qfilter == 1 && ql != 1)) return 0;
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

// block-wide exclusive scan of one int per thread; returns the total
__device__ __forceinline__ int block_scan(int x, int* sh, int& excl) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  int incl = x;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) sh[w] = incl;
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) {
    const int t = sh[i];
    before += i < w ? t : 0;
    total += t;
  }
  __syncthreads();  // sh is reused by the next scan
  excl = before + incl - x;
  return __builtin_amdgcn_readfirstlane(total);
}

// Device-scope coherent 8-byte accesses (relaxed agent-scope atomics:
// global_store / global_load with the device scope bits).
__device__ __forceinline__ void st_agent(void* p, uint64_t x) {
  __hip_atomic_store(static_cast<uint64_t*>(p), x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_agent(const void* p) {
  return __hip_atomic_load(static_cast<uint64_t*>(const_cast<void*>(p)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// A long pair whose piece partial this workgroup stored: its partial slots
// [slot0, slot0 + np) and the first output row of its heads.
struct PieceRun {
  int v;
  int slot0, np;
  int64_t qrow0;
};

// The merge of every piece of r, by the workgroup that arrived last: thread
// tid owns (head, 4 output dims) entries tid, tid + kBlock, ...; MB pieces'
// loads are issued before any is consumed (indices past the last piece
// re-read it and are dropped: no load under a branch), running max per head.
template <typename T, int G, int D, int MB>
__device__ __forceinline__ void merge_pieces(const AttnArgs& a, const DynArgs& k,
                                             const PieceRun& r, int tid) {
  T* __restrict__ out = static_cast<T*>(a.out);
  for (int idx = tid; idx < G * D / 4; idx += kBlock) {
    const int head = idx / (D / 4);
    const int d0 = (idx - head * (D / 4)) * 4;
    float M = -INFINITY, L = 0.f;
    floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int pb = 0; pb < r.np; pb += MB) {
      uint64_t mlr[MB], oor[MB];
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        const int64_t sl = r.slot0 + min(pb + j, r.np - 1);
        mlr[j] = ld_agent(k.part_ml + (sl * G + head) * 2);
        oor[j] = ld_agent(k.part_o + (sl * G + head) * D + d0);
      }
#pragma unroll
      for (int j = 0; j < MB; ++j) {
        float2 ml;
        half4 oo;
        __builtin_memcpy(&ml, &mlr[j], 8);
        __builtin_memcpy(&oo, &oor[j], 8);
        if (pb + j >= r.np || ml.x == -INFINITY) continue;
        const float Mn = fmaxf(M, ml.x);
        const float sa = exp2f(M - Mn);
        const float wl = ml.y * exp2f(ml.x - Mn);  // this piece's weight
        L = L * sa + wl;
        acc = acc * sa +
              floatx4{(float)oo[0], (float)oo[1], (float)oo[2], (float)oo[3]} * wl;
        M = Mn;
      }
    }
    const int64_t qrow = r.qrow0 + head;
    const float inv = L > 0.f ? 1.f / L : 0.f;
    T* dst = out + qrow * D + d0;
    dst[0] = (T)(acc[0] * inv);
    dst[1] = (T)(acc[1] * inv);
    dst[2] = (T)(acc[2] * inv);
    dst[3] = (T)(acc[3] * inv);
    if (d0 == 0 && a.lse) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2f : INFINITY;
  }
}

template <typename T, int G, int D>
__device__ __forceinline__ void merge_run(const AttnArgs& a, const DynArgs& k, const PieceRun& r,
                                          int tid) {
  if (r.np <= 2)
    merge_pieces<T, G, D, 2>(a, k, r, tid);
  else if (r.np <= 4)
    merge_pieces<T, G, D, 4>(a, k, r, tid);
  else
    merge_pieces<T, G, D, 8>(a, k, r, tid);
}

// One item of the list: pair v, chunks [c_lo, c_hi) of its n, whole or a
// piece.
struct Item {
  int v, c_lo, c_hi, n, np, j, kv_len;
};
// (read from LDS, the same for every lane: kept in scalar registers)
__device__ __forceinline__ Item decode_item(const uint32_t* items, const int* kvl, int i, int P) {
  const uint32_t it = __builtin_amdgcn_readfirstlane(items[i]);
  Item x;
  x.v = (int)(it >> 16);
  x.j = (int)(it & 0xffffu);
  x.kv_len = __builtin_amdgcn_readfirstlane(kvl[x.v]);
  x.n = x.kv_len > 0 ? (x.kv_len + kChunk - 1) / kChunk : 1;
  x.np = x.n > P ? (x.n + P - 1) / P : 1;
  x.c_lo = (int)((int64_t)x.j * x.n / x.np);
  x.c_hi = (int)((int64_t)(x.j + 1) * x.n / x.np);
  return x;
}

template <typename T, int D, int NT, int PF, bool OFF64>
__global__ __launch_bounds__(kBlock, 1) void decode_dyn_kernel(AttnArgs a, DynArgs k) {
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
  __shared__ uint32_t items[kDynItemCap];  // (pair << 16) | piece
  __shared__ int kvl[kDynMaxSeq];          // clamped context of each pair
  __shared__ int sh_cls[kClasses][kWaves];
  __shared__ int sh_base[kClasses];
  __shared__ int sh_scan[kWaves];
  __shared__ int s_grab, s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int grp = lane >> 4;
  const int l16 = lane & 15;
  const int wg = blockIdx.x;
  const int W = gridDim.x;
  const int V = a.n_seq * a.hkv;

  // ---- the work list (identical in every workgroup) ----
  int nch[2], kvv[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int v = b * kBlock + tid;
    nch[b] = 0;
    kvv[b] = 0;
    if (v < V) nch[b] = dyn_chunks(a, v, kvv[b]);
  }
  int unused;
  const int total_chunks = block_scan(nch[0] + nch[1], sh_scan, unused);
  // piece length: at least k.piece, and long enough that the list fits
  int P = k.piece;
  const int room = kDynItemCap - V;
  if ((int64_t)P * room < total_chunks) P = (total_chunks + room - 1) / room;
  const int lgP = 31 - __builtin_clz(P);
  int A = 0;  // pieces so far
  int run_c[kClasses];
#pragma unroll
  for (int c = 0; c < kClasses; ++c) run_c[c] = 0;
  int ppos[2] = {0, 0}, npc[2] = {0, 0}, cls[2] = {-1, -1}, rk[2] = {0, 0};
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    if (b * kBlock >= V) break;  // uniform
    const int n = nch[b];
    npc[b] = n > P ? (n + P - 1) / P : 0;
    int ex;
    const int tp = block_scan(npc[b], sh_scan, ex);
    ppos[b] = A + ex;
    A += tp;
    const bool whole = n > 0 && n <= P;
    const int c = whole ? min(kClasses - 1, lgP - (31 - __builtin_clz(n))) : -1;
    cls[b] = c;
    int myrank = 0;
#pragma unroll
    for (int cc = 0; cc < kClasses; ++cc) {
      const uint64_t m = __ballot(c == cc);
      if (c == cc) myrank = __popcll(m & ((1ull << lane) - 1));
      if (lane == 0) sh_cls[cc][w] = __popcll(m);
    }
    __syncthreads();
#pragma unroll
    for (int cc = 0; cc < kClasses; ++cc) {
      int tc = 0, before = 0;
#pragma unroll
      for (int ww = 0; ww < kWaves; ++ww) {
        const int t = sh_cls[cc][ww];
        tc += t;
        before += ww < w ? t : 0;
      }
      if (cc == c) rk[b] = run_c[cc] + before + myrank;
      run_c[cc] += tc;
    }
    __syncthreads();
  }
  int n_items = A;
#pragma unroll
  for (int c = 0; c < kClasses; ++c) {
    if (tid == 0) sh_base[c] = n_items;
    n_items += run_c[c];
  }
  __syncthreads();
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int v = b * kBlock + tid;
    if (v >= V) continue;
    kvl[v] = kvv[b];
    if (npc[b] > 0) {
      for (int j = 0; j < npc[b]; ++j) items[ppos[b] + j] = ((uint32_t)v << 16) | (uint32_t)j;
    } else if (cls[b] >= 0) {
      items[sh_base[cls[b]] + rk[b]] = (uint32_t)v << 16;
    }
  }
  __syncthreads();

  // ---- the schedule: static items wg and 2W - 1 - wg, then draws ----
  const int total_draws = max(0, n_items - 2 * W) + W;
  int q0 = wg < n_items ? wg : -1;
  int q1 = 2 * W - 1 - wg < n_items ? 2 * W - 1 - wg : -1;
  if (q0 < 0) {
    // no item: the one empty draw every workgroup makes
    if (tid == 0) {
      const int d = __hip_atomic_fetch_add(k.ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == total_draws - 1)
        __hip_atomic_store(k.ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }
  bool drawing = true;

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

  Item it = decode_item(items, kvl, q0, P);
  v8 qf[NT][D / 32];
  {
    const int s = it.v / a.hkv;
    const int qtok = a.qloc ? ld_meta(a.qloc, s) : s;
    load_q<T, D, NT>(qf, q, (int64_t)qtok * a.hq + (it.v - s * a.hkv) * G, grp, l16);
  }
  bool prestaged = false;  // this item's first table window is in LDS
  PieceRun pend;           // piece whose partial was stored, arrival not yet counted
  pend.v = -1;
  for (;;) {
    const int s = it.v / a.hkv;
    const int kvh = it.v - s * a.hkv;
    const int qtok = a.qloc ? ld_meta(a.qloc, s) : s;
    const int64_t qrow0 = (int64_t)qtok * a.hq + kvh * G;
    const int tok_lo = it.c_lo * kChunk;
    const int tok_hi = min(it.c_hi * kChunk, it.kv_len);
    const bool whole = it.np == 1;
    // the next draw, read at this item's end
    int d = 0;
    if (drawing && tid == 0)
      d = __hip_atomic_fetch_add(k.ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    NewRow nr;  // no appended row: the library appends before this kernel
    nr.pos = -1;
    nr.lds = nullptr;
    pv.head_off = (int64_t)kvh * D * 2;
    const int32_t* __restrict__ table = a.block_tables + (int64_t)s * a.max_blk;
    WaveState<NT, DT> st;
    st.reset();
    for (int lo = tok_lo; lo < tok_hi; lo += win) {
      cx.seg_lo = lo;
      cx.seg_hi = min(lo + win, tok_hi);
      cx.blk_lo = lo >> a.bs_shift;
      const int nblk = ((cx.seg_hi - 1) >> a.bs_shift) + 1 - cx.blk_lo;
      __syncthreads();  // previous window's table and slices no longer read
      if (!(prestaged && lo == tok_lo)) {  // else staged during the previous item's merge
        for (int i = tid; i < nblk; i += kBlock) tbl[i] = table[cx.blk_lo + i];
      }
      __syncthreads();
      run_chunks<T, D, NT, PF, OFF64, false>(w, kWaves, cx, pv, qf, st, bad_block, nr);
    }

    // ---- every chunk load has been consumed: this thread's stores of the
    // pending piece and the draw have completed; after the barrier
    // everyone's have, and the pending piece's arrival is counted (issued
    // before the next item's loads, so its result does not wait for them)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (tid == 0) s_grab = d;
    __syncthreads();
    int arrived = 0;
    if (pend.v >= 0 && tid == 0)
      arrived = __hip_atomic_fetch_add(k.ctr + 1 + pend.v, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
    // ---- the queue: q1, then the drawn item
    int drawn = -1;
    if (drawing) {
      const int dd = __builtin_amdgcn_readfirstlane(s_grab);
      if (2 * W + dd < n_items) {
        drawn = 2 * W + dd;
      } else {
        drawing = false;
        if (dd == total_draws - 1 && tid == 0)
          __hip_atomic_store(k.ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    const int cur = q0;
    q0 = q1 >= 0 ? q1 : drawn;
    q1 = q1 >= 0 ? drawn : -1;
    const bool has_next = q0 >= 0;

    // ---- the next item's Q and first table window are requested now (qf
    // is free once this item has streamed; the table is written to LDS
    // after the merge). Issued whether or not there is a next item (then
    // they re-read this one's), so no load sits under a branch.
    int tpref, n_nblk;
    {
    const Item nx = decode_item(items, kvl, has_next ? q0 : cur, P);
    const int s_n = nx.v / a.hkv;
    const int kvh_n = nx.v - s_n * a.hkv;
    const int qtok_n = a.qloc ? ld_meta(a.qloc, s_n) : s_n;
    load_q<T, D, NT>(qf, q, (int64_t)qtok_n * a.hq + kvh_n * G, grp, l16);
    const int tok_lo_n = nx.c_lo * kChunk;
    const int tok_hi_n = min(nx.c_hi * kChunk, nx.kv_len);
    const int blk_lo_n = tok_lo_n >> a.bs_shift;
    n_nblk = has_next && tok_hi_n > tok_lo_n
                 ? ((min(tok_lo_n + win, tok_hi_n) - 1) >> a.bs_shift) + 1 - blk_lo_n
                 : 0;
    // max_blk >= 1 for this kernel: entry 0 of the row is always readable
    tpref = a.block_tables[(int64_t)s_n * a.max_blk +
                           max(0, min(blk_lo_n + tid, blk_lo_n + n_nblk - 1))];
    }

    // ---- merge the wavefronts' states through LDS ----
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) st.l[nt] = head_lanes_sum(st.l[nt]);
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
    if (pend.v >= 0 && tid == 0) {
      s_last = arrived == pend.np - 1;
      if (s_last)
        __hip_atomic_store(k.ctr + 1 + pend.v, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
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
      const float inv = L > 0.f ? 1.f / L : 0.f;
      if (whole) {
        const int64_t qrow = qrow0 + head;
        T* dst = out + qrow * D + d0;
        dst[0] = (T)(acc[0] * inv);
        dst[1] = (T)(acc[1] * inv);
        dst[2] = (T)(acc[2] * inv);
        dst[3] = (T)(acc[3] * inv);
        if (d0 == 0 && a.lse) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2f : INFINITY;
      } else {
        // normalised by its own sum (a weighted mean of value rows, so its
        // range is theirs) and rounded to fp16: half the partial traffic
        const half4 o16 = half4{(_Float16)(acc[0] * inv), (_Float16)(acc[1] * inv),
                                (_Float16)(acc[2] * inv), (_Float16)(acc[3] * inv)};
        uint64_t bits;
        __builtin_memcpy(&bits, &o16, 8);
        st_agent(k.part_o + ((int64_t)cur * G + head) * D + d0, bits);
        if (d0 == 0) {
          const float2 ml = make_float2(M, L);
          __builtin_memcpy(&bits, &ml, 8);
          st_agent(k.part_ml + ((int64_t)cur * G + head) * 2, bits);
        }
      }
    }
    // ---- the previous piece: merged here if this workgroup arrived last
    if (pend.v >= 0) {
      if (s_last) merge_run<T, G, D>(a, k, pend, tid);
      pend.v = -1;
    }
    if (!whole) {
      pend.v = it.v;
      pend.slot0 = cur - it.j;
      pend.np = it.np;
      pend.qrow0 = qrow0;
    }
    __syncthreads();  // LDS merge area and table are free
    if (!has_next) break;
    if (tid < n_nblk) tbl[tid] = tpref;  // published by the window loop's first barrier
    prestaged = true;
    it = decode_item(items, kvl, q0, P);
  }
  // ---- the last piece's arrival, now
  if (pend.v >= 0) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      const int arrived = __hip_atomic_fetch_add(k.ctr + 1 + pend.v, 1, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
      s_last = arrived == pend.np - 1;
      if (s_last)
        __hip_atomic_store(k.ctr + 1 + pend.v, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (s_last) merge_run<T, G, D>(a, k, pend, tid);
  }
  if (bad_block && a.status) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
}

template <typename T, int D, int NT, int PF, bool OFF64>
int launch_v(const AttnArgs& a, const DynArgs& k, hipStream_t stream) {
  hipLaunchKernelGGL((decode_dyn_kernel<T, D, NT, PF, OFF64>), dim3(device_cu_count()),
                     dim3(kBlock), 0, stream, a, k);
  return check_launch("decode_dyn_kernel");
}

template <typename T, bool OFF64>
int launch_t(const AttnArgs& a, const DynArgs& k, hipStream_t stream) {
  const int nt = a.group / 16;
  // <T, D, NT, PF, OFF64>: two wavefronts per SIMD; the D = 128 variants
  // have room for one chunk in flight per wavefront, the D = 64 ones for two
  if (a.d == 64 && nt == 1) return launch_v<T, 64, 1, 2, OFF64>(a, k, stream);
  if (a.d == 64 && nt == 2) return launch_v<T, 64, 2, 2, OFF64>(a, k, stream);
  if (a.d == 128 && nt == 1) return launch_v<T, 128, 1, 1, OFF64>(a, k, stream);
  if (a.d == 128 && nt == 2) return launch_v<T, 128, 2, 1, OFF64>(a, k, stream);
  return fail(PKV_ERR_UNSUPPORTED, "decode_dyn: d=%d group=%d", a.d, a.group);
}

}  // namespace

int launch_decode_dyn(const AttnArgs& a, const DynArgs& k, int dtype, hipStream_t stream) {
  if (a.num_blocks >= (int64_t(1) << 31))
    return fail(PKV_ERR_UNSUPPORTED, "decode_dyn: %lld blocks", (long long)a.num_blocks);
  if ((int64_t)a.n_seq * a.hkv > kDynMaxSeq)
    return fail(PKV_ERR_UNSUPPORTED, "decode_dyn: %d pairs", a.n_seq * a.hkv);
  const bool off64 = pool_needs_off64(a);
  if (dtype == PKV_DTYPE_BF16)
    return off64 ? launch_t<bf16, true>(a, k, stream) : launch_t<bf16, false>(a, k, stream);
  if (dtype == PKV_DTYPE_F16)
    return off64 ? launch_t<f16, true>(a, k, stream) : launch_t<f16, false>(a, k, stream);
  return fail(PKV_ERR_UNSUPPORTED, "decode_dyn: dtype %d", dtype);
}

}  // namespace pkv
