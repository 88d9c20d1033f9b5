// Paged MQA decode, persistent form: one workgroup per CU (two at head dim
// 64), each owning an equal share of all sequences' work.
//
// Every (sequence, kv head) pair v with a query is laid end to end on a cost
// line as K overhead units (its Q load, table slice, wavefront merge and
// output, worth about K chunks of streaming) followed by its n_v 32-token
// chunks. With C units in total and W workgroups, workgroup w owns units
// [R(w), R(w+1)), R(w) = floor(w C / W), and processes the chunks among
// them. Every workgroup gets the same amount of work whatever the length
// distribution (one that covers many short sequences streams fewer chunks):
//   - a sequence that lies entirely inside one share is finished in place
//     (its wavefronts' states are merged through LDS and written out);
//   - a sequence cut by share boundaries gets one partial (m, l, O/l) per
//     workgroup that touches it (its first or last segment there, so at most
//     two per workgroup), written through to memory; each contributor then
//     counts itself in on the sequence's arrival counter, and the one that
//     completes the count merges every partial (in contributor order) and
//     writes the row. Nothing waits on another workgroup, so the scheme
//     cannot deadlock whatever the residency.
// The per-chunk pipeline is mfma_decode_common.h. Semantics are those of
// pagedattn.forward (kernels/pagedattn/pagedattn.cu:142-447) for q_len = 1.
#include "mfma_decode_common.h"
#include "prefill_mfma.h"

namespace pkv {
namespace {

using namespace mfma;

// Wavefronts per workgroup: at D = 64, 4 (two workgroups per CU; an
// 8-wavefront combination of 16 heads x 64 dims would leave threads without a
// column); at D = 128, 4 for a batch of decode sequences alone (one
// workgroup per CU, at most 256 VGPRs) and 8 for the decode part of a mixed
// batch, the size of the one-launch mixed kernel's workgroups (so that both
// forms of a mixed call give the same results).
constexpr int sk_waves(int d) { return d == 128 ? 8 : 4; }

// Chunks of virtual sequence v (= sequence * hkv + kv head) and its clamped
// context, from its query_start_loc pair (q0, q1; 0, 1 without
// query_start_loc) and seq_len: 0 chunks when the sequence has no query this
// step, at least 1 otherwise (an empty context still owes a zero row and
// lse = +inf); a malformed pair has been flagged by the scan (scan_desc)
struct SeqDesc {
  int n, kv_len;
};
__device__ __forceinline__ SeqDesc seq_desc(const AttnArgs& a, int q0, int q1, int kl) {
  SeqDesc d{0, 0};
  if (a.qloc && (q1 - q0 <= 0 || q0 < 0 || q1 > a.n_tokens ||
                 (a.qfilter == 1 && q1 - q0 != 1)))
    return d;
  const int cap = a.max_blk << a.bs_shift;
  kl = kl < cap ? kl : cap;
  d.kv_len = kl > 0 ? kl : 0;
  d.n = d.kv_len > 0 ? (d.kv_len + kChunk - 1) / kChunk : 1;
  return d;
}
// The three loads are issued together whether or not query_start_loc is
// given (without it, `alt` - any buffer of at least s + 2 ints - is read
// and ignored), so they cost one round trip.
__device__ __forceinline__ SeqDesc load_desc(const AttnArgs& a, int v, const int32_t* alt) {
  const int s = v / a.hkv;
  const int32_t* qsrc = a.qloc ? a.qloc : alt;
  const int kl = ld_meta(a.seq_lens, s);
  const int q0 = ld_meta(qsrc, s);
  const int q1 = ld_meta(qsrc, s + 1);
  return seq_desc(a, a.qloc ? q0 : 0, a.qloc ? q1 : 1, kl);
}

// The scan's view of pair v: its three metadata loads issued together
// (vector loads, one round trip) and its query token; a malformed query
// range is flagged once (by workgroup 0).
struct ScanDesc {
  SeqDesc d;
  int q0;  // first query token (its row of q / out)
};
__device__ __forceinline__ ScanDesc scan_desc(const AttnArgs& a, int v, const int32_t* alt,
                                              bool flagger) {
  const int s = v / a.hkv;
  const int32_t* qsrc = a.qloc ? a.qloc : alt;
  const int kl = a.seq_lens[s];
  const int q0 = qsrc[s];
  const int q1 = qsrc[a.qloc ? s + 1 : s];
  ScanDesc r;
  r.q0 = a.qloc ? q0 : s;
  const int ql = a.qloc ? q1 - q0 : 1;
  if (a.qloc && ql > 0 && !(a.qfilter == 1 && ql != 1) && (q0 < 0 || q0 + ql > a.n_tokens) &&
      a.status && flagger)
    atomicOr(a.status, PKV_STATUS_BAD_QLOC);
  r.d = seq_desc(a, r.q0, a.qloc ? q1 : s + 1, kl);
  return r;
}

// first chunk of workgroup w's share, and the workgroup owning chunk x
__device__ __forceinline__ int share_start(int w, int C, int W) {
  return (int)((int64_t)w * C / W);
}
__device__ __forceinline__ int share_owner(int x, int C, int W) {
  return (int)(((int64_t)(x + 1) * W - 1) / C);
}

// Cost of virtual sequence v on the share line: 0 without a query, else
// seg_cost overhead units plus its chunks.
__device__ __forceinline__ int sk_cost(int n, int seg_cost) { return n > 0 ? n + seg_cost : 0; }

__device__ __forceinline__ uint64_t ld_agent64(const void* p) {
  return __hip_atomic_load(static_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Partial slot of contributor ww of a sequence cut over [w_first, w_last]:
// the sequence is the first segment of every contributor but w_first, whose
// slot is 2 w_first + r_slot (r_slot = 1 when its share starts with an
// earlier sequence).
__device__ __forceinline__ int64_t cut_slot(int ww, int w_first, int r_slot) {
  return ww == w_first ? 2 * (int64_t)ww + r_slot : 2 * (int64_t)ww;
}

// Combination of every partial of a cut sequence, in contributor order (so
// the result does not depend on which contributor merges): thread tid owns
// head tid / TPH and the float4 columns cq + TPH q, the (max, sum) pair of
// its head is read once per contributor, and every load of a batch of kMB
// contributors is issued before any is consumed. Loads are device-coherent (they bypass this XCD's L2:
// the partials were written through from other XCDs during this launch).
template <typename T, int G, int D, int NW>
__device__ __forceinline__ void merge_cut(const AttnArgs& a, const SkArgs& k, int w_first,
                                          int w_last, int r_slot, int64_t qrow0, int tid) {
  constexpr int kBlock = 64 * NW;
  constexpr int TPH = kBlock / G;
  constexpr int NQ = D / (4 * TPH);
  constexpr int kMB = 4;
  const int head = tid / TPH;
  const int cq = tid - head * TPH;
  float M = -INFINITY, L = 0.f;
  floatx4 acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
  for (int wb = w_first; wb <= w_last; wb += kMB) {
    uint64_t mlr[kMB], oor[kMB][NQ];
#pragma unroll
    for (int j = 0; j < kMB; ++j) {
      const int64_t row = cut_slot(min(wb + j, w_last), w_first, r_slot) * G + head;
      mlr[j] = ld_agent64(k.part_ml + row * 2);
#pragma unroll
      for (int q = 0; q < NQ; ++q) oor[j][q] = ld_agent64(k.part_o + row * D + 4 * (cq + TPH * q));
    }
#pragma unroll
    for (int j = 0; j < kMB; ++j) {
      float2 ml;
      __builtin_memcpy(&ml, &mlr[j], 8);
      if (wb + j > w_last || ml.x == -INFINITY) continue;
      const float Mn = fmaxf(M, ml.x);
      const float sa = exp2f(M - Mn);
      const float wl = ml.y * exp2f(ml.x - Mn);  // this partial's weight
      L = L * sa + wl;
#pragma unroll
      for (int q = 0; q < NQ; ++q) acc[q] = acc[q] * sa + unpack4<T>(oor[j][q]) * wl;
      M = Mn;
    }
  }
  const int64_t qrow = qrow0 + head;
  const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    T* dst = static_cast<T*>(a.out) + qrow * D + 4 * (cq + TPH * q);
    dst[0] = (T)(acc[q][0] * inv);
    dst[1] = (T)(acc[q][1] * inv);
    dst[2] = (T)(acc[q][2] * inv);
    dst[3] = (T)(acc[q][3] * inv);
  }
  if (cq == 0 && a.lse) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2f : INFINITY;
}

// Workgroup geometry and LDS sizes of the persistent kernel with NW
// wavefronts per workgroup.
template <int D, int NT, int NW>
struct SkGeo {
  static constexpr int kWaves = NW;
  static constexpr int kBlock = 64 * kWaves;
  static constexpr int G = 16 * NT;
  static constexpr int WAVE_BYTES = 2 * ChunkGeo<D>::BYTES;
  template <typename S>
  using Combine = WaveCombine16<S, G, D, kWaves, kBlock>;
  static constexpr int MERGE_BYTES = kWaves * G * Combine<bf16>::OPITCH * 2;
  static constexpr int MAIN_BYTES = kWaves * WAVE_BYTES;
  // the wavefronts' chunk slices while streaming, the merge area after
  static constexpr int LDS_BYTES = MAIN_BYTES > MERGE_BYTES ? MAIN_BYTES : MERGE_BYTES;
  static constexpr int ROW_BYTES = 2 * D * 2;  // an appended K and V row (16-bit)
};

// LDS of one persistent workgroup: pointers to arrays the kernel declares as
// separate __shared__ objects (so the compiler keeps their accesses apart).
template <int D, int NT>
struct SkLds {
  char* lds;                    // SkGeo::LDS_BYTES, 16-byte aligned
  float (*ml_lds)[16 * NT][2];  // [kWaves]: the wavefronts' (max, sum) per head
  int* tbl;                     // kTblCap: the segment's table window
  int* scan_sh;                 // kBlock: block scans
  int* sv;                      // 6: the share's first sequence (v, g0, n, kv_len, query
                                // token) and the last-arriver flag
  char* nrow;                   // APP: the segment's appended row, K then V (ROW_BYTES)
};

// Persistent workgroup `wg` of k.n_wg, NW wavefronts. APP: a mixed-batch launch whose
// table append runs in the same grid (the prefill workgroups write the
// decode rows): each sequence's new row, at position new_pos[s], is taken
// from k_new / v_new (the sequence's query token) in place of its pool row,
// which may not be written yet; this workgroup writes no pool row.
template <typename T, int D, int NT, int PF, bool HALVES, bool KV8, bool APP, int NW>
__device__ __forceinline__ void decode_sk_body(AttnArgs a, SkArgs k, int wg,
                                               const SkLds<D, NT>& sm) {
  using SG = SkGeo<D, NT, NW>;
  constexpr int kWaves = SG::kWaves;
  constexpr int kBlock = SG::kBlock;
  using Geo = ChunkGeo<D>;
  using v8 = typename Ops<T>::v8;
  constexpr int G = SG::G;
  constexpr int DT = D / 16;
  constexpr int WAVE_BYTES = SG::WAVE_BYTES;
  using Combine = typename SG::template Combine<T>;
  char* const lds = sm.lds;
  float(*const ml_lds)[G][2] = sm.ml_lds;
  int* const tbl = sm.tbl;
  int* const scan_sh = sm.scan_sh;
  int& s_v0 = sm.sv[0];
  int& s_g0 = sm.sv[1];
  int& s_n0 = sm.sv[2];
  int& s_kl0 = sm.sv[3];
  int& s_q0 = sm.sv[4];
  int& s_last = sm.sv[5];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int grp = lane >> 4;
  const int l16 = lane & 15;
  const int V = a.n_seq * a.hkv;

  // ---- total cost C, then the sequence whose cost interval holds this
  // share's start (the first pass's values are kept when V fits one block)
  const int K = k.seg_cost;
  int C = 0;
  int n_mine = 0, ex_mine = 0;
  ScanDesc sd_mine{};
  const int32_t* alt = reinterpret_cast<const int32_t*>(k.recs);
  for (int base = 0; base < V; base += kBlock) {
    const ScanDesc sd = scan_desc(a, min(base + tid, V - 1), alt, wg == 0);
    const int n = base + tid < V ? sk_cost(sd.d.n, K) : 0;
    int ex;
    C += block_scan<kWaves>(n, scan_sh, ex);
    n_mine = n;
    ex_mine = ex;
    sd_mine = sd;
  }
  // at most one share per unit, so that every share is non-empty
  const int W = k.n_wg < C ? k.n_wg : C;
  if (wg >= W) return;
  const int start = share_start(wg, C, W);
  const int end = share_start(wg + 1, C, W);
  if (tid == 0) s_v0 = -1;
  __syncthreads();
  // the pair whose interval holds the share's start, with its metadata (so
  // the segment loop starts without reloading it)
  if (V <= kBlock) {
    if (n_mine > 0 && ex_mine <= start && start < ex_mine + n_mine) {
      s_v0 = tid;
      s_g0 = ex_mine;
      s_n0 = sd_mine.d.n;
      s_kl0 = sd_mine.d.kv_len;
      s_q0 = sd_mine.q0;
    }
  } else {
    int run = 0;
    for (int base = 0; base < V; base += kBlock) {
      const int v = base + tid;
      const ScanDesc sd = scan_desc(a, min(v, V - 1), alt, wg == 0);
      const int n = v < V ? sk_cost(sd.d.n, K) : 0;
      int ex;
      const int tot = block_scan<kWaves>(n, scan_sh, ex);
      if (n > 0 && run + ex <= start && start < run + ex + n) {
        s_v0 = v;
        s_g0 = run + ex;
        s_n0 = sd.d.n;
        s_kl0 = sd.d.kv_len;
        s_q0 = sd.q0;
      }
      run += tot;
      __syncthreads();
      if (s_v0 >= 0) break;
    }
  }
  __syncthreads();

  PoolView pv;
  pv.kbase = static_cast<const char*>(a.k_pool);
  pv.vbase = static_cast<const char*>(a.v_pool);
  pv.row_stride = (int64_t)a.hkv * D * (KV8 ? 1 : 2);
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
  T* ob = reinterpret_cast<T*>(lds);
  // kTblCap - 1 blocks of tokens: a window that starts inside a block still
  // touches at most kTblCap table entries
  const int win = (kTblCap - 1) << a.bs_shift;

  // uniform across the workgroup: scalar registers for the segment loop
  int v = __builtin_amdgcn_readfirstlane(s_v0);
  int g0 = __builtin_amdgcn_readfirstlane(s_g0);  // cost position where v's interval starts
  SeqDesc dsc;  // n > 0: the share's start lies in v's chunks
  dsc.n = __builtin_amdgcn_readfirstlane(s_n0);
  dsc.kv_len = __builtin_amdgcn_readfirstlane(s_kl0);
  v8 qf[NT][D / 32];
  // APP: the segment's appended row (its pieces in registers until staged in
  // LDS with the segment's first table window) and its position. Requested
  // for every segment, with the segment's Q: it costs no extra round trip.
  u32x4 nrp{};
  int npos = -1;
  {
    const int s = v / a.hkv;
    const int qtok = __builtin_amdgcn_readfirstlane(s_q0);
    load_q<T, D, NT>(qf, q, (int64_t)qtok * a.hq + (v - s * a.hkv) * G, grp, l16);
    if constexpr (APP) {
      nrp = load_new_row<D>(a, qtok, v - s * a.hkv, tid);
      npos = ld_meta(a.new_pos, s);
    }
  }
  bool first = true;
  bool prestaged = false;  // this segment's first table window (and new row) is in LDS
  // Segment loop: sequence v's chunks sit at units [g0 + K, g0 + K + n) of
  // the cost line; the share's chunks are those among [start, end). Once a
  // segment has streamed, the next one's Q and first table window are loaded
  // while this one's wavefront states are merged and written, so the next
  // segment starts streaming without a dependent load.
  for (;;) {
    const int n = dsc.n;
    const int kv_len = dsc.kv_len;
    const int c0 = max(0, start - (g0 + K));
    const int c1 = min(n, end - (g0 + K));
    // a share shorter than seg_cost can lie entirely in v's overhead units:
    // it owns none of v's chunks (nor any later ones), so it is no
    // contributor and has nothing to do
    if (c1 <= c0) break;
    const bool whole = c0 == 0 && c1 == n;
    const int s = v / a.hkv;
    const int kvh = v - s * a.hkv;
    const int qtok = a.qloc ? ld_meta(a.qloc, s) : s;
    const int64_t qrow0 = (int64_t)qtok * a.hq + kvh * G;
    const int tok_lo = c0 * kChunk;
    const int tok_hi = min(c1 * kChunk, kv_len);
    // the next sequence's metadata, in flight while this segment streams
    const bool more = v + 1 < V;
    int nq0 = 0, nq1 = 1, nkl = 0;
    if (more) {
      const int sn = (v + 1) / a.hkv;
      if (a.qloc) {
        nq0 = ld_meta(a.qloc, sn);
        nq1 = ld_meta(a.qloc, sn + 1);
      }
      nkl = ld_meta(a.seq_lens, sn);
    }

    NewRow nr;  // APP: staged over its pool row where it falls in this segment
    nr.pos = APP ? npos : -1;
    nr.lds = sm.nrow;
    pv.head_off = (int64_t)kvh * D * (KV8 ? 1 : 2);
    const int32_t* __restrict__ table = a.block_tables + (int64_t)s * a.max_blk;
    WaveState<NT, DT> st;
    st.reset();
    for (int lo = tok_lo; lo < tok_hi; lo += win) {
      cx.seg_lo = lo;
      cx.seg_hi = min(lo + win, tok_hi);
      cx.blk_lo = lo >> a.bs_shift;
      const int nblk = ((cx.seg_hi - 1) >> a.bs_shift) + 1 - cx.blk_lo;
      __syncthreads();  // previous window's table and slices no longer read
      if (!(prestaged && lo == tok_lo)) {  // else staged during the previous segment's merge
        for (int i = tid; i < nblk; i += kBlock) tbl[i] = table[cx.blk_lo + i];
        if (APP && lo == tok_lo) put_new_row<D>(sm.nrow, nrp, tid);
      }
      __syncthreads();
      run_chunks<T, D, NT, PF, HALVES, APP, KV8>(w, kWaves, cx, pv, qf, st, bad_block, nr);
    }

    // ---- the next segment: its Q and first table window are loaded now
    // (qf is free once this segment has streamed; the table is written to
    // LDS after the merge)
    int v_n = v + 1;
    const int g0_n = g0 + n + K;
    SeqDesc d_n = seq_desc(a, nq0, nq1, nkl);
    bool has_next = more && g0_n + K < end;
    while (has_next && d_n.n == 0) {  // sequences without a query cost nothing
      ++v_n;
      has_next = v_n < V;
      if (has_next) d_n = load_desc(a, v_n, reinterpret_cast<const int32_t*>(k.recs));
    }
    // Its first chunk is chunk 0 (g0_n + K lies past this segment's start).
    // The loads are issued whether or not there is a next segment (then
    // they re-read this one's rows, and are dropped): a load under a branch
    // would cost the chunk loop its exact wait counts.
    const int v_sel = has_next ? v_n : v;
    const int s_n = v_sel / a.hkv;
    const int kvh_n = v_sel - s_n * a.hkv;
    const int qtok_n = a.qloc ? ld_meta(a.qloc, s_n) : s_n;
    load_q<T, D, NT>(qf, q, (int64_t)qtok_n * a.hq + kvh_n * G, grp, l16);
    int npos_n = -1;
    if constexpr (APP) {
      nrp = load_new_row<D>(a, qtok_n, kvh_n, tid);
      npos_n = ld_meta(a.new_pos, s_n);
    }
    const int c1_n = min(d_n.n, end - (g0_n + K));
    const int tok_hi_n = min(c1_n * kChunk, d_n.kv_len);
    const int n_nblk =
        has_next && tok_hi_n > 0 ? ((min(win, tok_hi_n) - 1) >> a.bs_shift) + 1 : 0;
    // max_blk >= 1 for this kernel: entry 0 of the row is always readable
    const int tpref =
        a.block_tables[(int64_t)s_n * a.max_blk + max(0, min(tid, n_nblk - 1))];

    // ---- merge the wavefronts' states through LDS ----
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      st.l[nt] = head_lanes_sum(st.l[nt]);
    }
    __syncthreads();
    // each wavefront's O / l rounded to T (see WaveCombine16)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float il = st.l[nt] > 0.f ? 1.f / st.l[nt] : 0.f;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<uint64_t*>(ob + (w * G + 16 * nt + l16) * Combine::OPITCH + 16 * dt +
                                     4 * grp) = pack4<T>(st.o[nt][dt], il);
    }
    if (grp == 0) {
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        ml_lds[w][16 * nt + l16][0] = st.m[nt];
        ml_lds[w][16 * nt + l16][1] = st.l[nt];
      }
    }
    __syncthreads();
    const int slot = 2 * wg + (first ? 0 : 1);
    {
      Combine cb;
      cb.run(ob, ml_lds, tid);
      const float inv = cb.inv;
      if (whole) {
        const int64_t qrow = qrow0 + cb.head;
#pragma unroll
        for (int q = 0; q < cb.NQ; ++q) {
          T* dst = out + qrow * D + cb.col(q);
          dst[0] = (T)(cb.acc[q][0] * inv);
          dst[1] = (T)(cb.acc[q][1] * inv);
          dst[2] = (T)(cb.acc[q][2] * inv);
          dst[3] = (T)(cb.acc[q][3] * inv);
        }
        if (cb.cq == 0 && a.lse)
          a.lse[qrow] = cb.L > 0.f ? (cb.M + log2f(cb.L)) * kLn2f : INFINITY;
      } else {
        // normalised by its own sum (a weighted mean of value rows, so its
        // range is theirs) and rounded to T: half the partial traffic
        const int64_t prow = (int64_t)slot * G + cb.head;
#pragma unroll
        for (int q = 0; q < cb.NQ; ++q)
          // written through: the merging workgroup may sit on another XCD
          st_agent64(k.part_o + prow * D + cb.col(q), pack4<T>(cb.acc[q], inv));
        if (cb.cq == 0) {
          const float2 ml = make_float2(cb.M, cb.L);
          uint64_t b;
          __builtin_memcpy(&b, &ml, 8);
          st_agent64(k.part_ml + prow * 2, b);
        }
      }
    }

    if (!whole) {
      // once this workgroup's partial stores have completed, it counts
      // itself in on the sequence's arrival counter (the last int of its
      // record); the contributor that brings the count to the number of
      // contributors merges every partial and puts the counter back to
      // zero for the next call. No workgroup waits for another.
      const int w_first = share_owner(g0 + K, C, W);
      const int w_last = share_owner(g0 + K + n - 1, C, W);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (tid == 0) {
        int* ctr = reinterpret_cast<int*>(k.recs + v) + 3;
        const int old = fetch_add_agent(ctr, 1);
        s_last = old == w_last - w_first;
        if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // a dirty counter (start value c != 0) shows a value outside
        // [0, contributors) to at least one contributor
        if ((old < 0 || old > w_last - w_first) && a.status)
          atomicOr(a.status, PKV_STATUS_DIRTY_WORKSPACE);
      }
      __syncthreads();
      if (s_last)
        merge_cut<T, G, D, kWaves>(a, k, w_first, w_last, share_start(w_first, C, W) < g0 ? 1 : 0,
                           qrow0, tid);
    }
    __syncthreads();  // LDS merge area, table and row buffer are free
    if (!has_next) break;
    // published by the window loop's first barrier
    if (tid < n_nblk) tbl[tid] = tpref;
    if constexpr (APP) put_new_row<D>(sm.nrow, nrp, tid);
    prestaged = true;
    v = v_n;
    g0 = g0_n;
    dsc = d_n;
    npos = npos_n;
    first = false;
  }
  if (bad_block && a.status) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
}

template <typename T, int D, int NT, int PF, bool HALVES, bool KV8, int NW>
__global__ __launch_bounds__(64 * NW, 8 / NW) void decode_sk_kernel(AttnArgs a, SkArgs k) {
  using SG = SkGeo<D, NT, NW>;
  __shared__ __attribute__((aligned(16))) char lds[SG::LDS_BYTES];
  __shared__ float ml_lds[SG::kWaves][SG::G][2];
  __shared__ int tbl[kTblCap];
  __shared__ int scan_sh[SG::kBlock];
  __shared__ int sv[6];
  const SkLds<D, NT> sm{lds, ml_lds, tbl, scan_sh, sv, nullptr};
  decode_sk_body<T, D, NT, PF, HALVES, KV8, false, NW>(a, k, blockIdx.x, sm);
}

// A mixed batch in one launch (D = 128, 16-bit pools): workgroups
// [0, k.n_wg) are the persistent decode kernel's shares over the one-token
// sequences (ad: qfilter 1, each new row taken from k_new), the rest the
// prefill kernel's pair workgroups over the others, pair slot i % pre_slots
// of kv head i / pre_slots (ap: qfilter 2, with the fused append of every
// row of the batch). No workgroup uses what another writes in this launch:
// a decode share loads its new row's pool slot with the rest of the chunk
// (a prefill workgroup may be writing it at that moment) but replaces it in
// LDS with the row from k_new / v_new before any use, and the prefill pairs
// read their own new rows from k_new / v_new. Dispatched in order, the
// decode shares fill the CUs first,
// and each pair workgroup starts on a CU as soon as a share there has
// ended, so the prefill's prologue and the decode shares' uneven ends
// overlap instead of adding up across two launches. (Pair workgroups that
// walk several slots, so that the grid holds no empty ones, measured
// slower: the loop costs the kernel 10 spilled VGPRs.)
template <typename T, int NT, bool HALVES>
__global__ __launch_bounds__(kPBlock, 1) void mixed_sk_kernel(AttnArgs ad, SkArgs k, AttnArgs ap,
                                                              int pre_slots) {
  constexpr int D = 128;
  using SG = SkGeo<D, NT, sk_waves(D)>;
  static_assert(SG::kBlock == kPBlock, "one workgroup size for both parts");
  constexpr int kLdsBytes =
      SG::LDS_BYTES > PrefillLds<D>::kBufBytes ? SG::LDS_BYTES : PrefillLds<D>::kBufBytes;
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  __shared__ float ml_lds[SG::kWaves][SG::G][2];
  __shared__ int tbl[kTblCap];
  __shared__ int scan_sh[SG::kBlock];
  __shared__ int sv[6];
  __shared__ __attribute__((aligned(16))) char nrow[SG::ROW_BYTES];
  __shared__ int dl_seq[kPBlock], dl_tok[kPBlock];
  const int b = blockIdx.x;
  if (b < k.n_wg) {
    const SkLds<D, NT> sm{lds, ml_lds, tbl, scan_sh, sv, nrow};
    decode_sk_body<T, D, NT, 1, HALVES, false, true, sk_waves(D)>(ad, k, b, sm);
  } else {
    const PrefillLds<D> sm{lds, tbl, scan_sh, sv, dl_seq, dl_tok};
    const int i = b - k.n_wg;
    prefill_pair_body<T, D, NT, false, false>(ap, i % pre_slots, i / pre_slots, sm);
  }
}

template <typename T, int NT, bool HALVES>
int launch_mixed_v(const AttnArgs& ad, SkArgs k, const AttnArgs& ap, hipStream_t stream) {
  k.n_wg = sk_workgroups(128, 16 * NT);
  k.seg_cost = kSkSegCost128(sk_waves(128));
  const int64_t slots = prefill_slots(ap.n_tokens, ap.n_seq, ap.group);
  const int64_t grid = k.n_wg + slots * ap.hkv;
  if (grid > 0x7fffffff)
    return fail(PKV_ERR_UNSUPPORTED, "mixed_sk: %lld workgroups", (long long)grid);
  hipLaunchKernelGGL((mixed_sk_kernel<T, NT, HALVES>), dim3((unsigned)grid), dim3(kPBlock), 0,
                     stream, ad, k, ap, (int)slots);
  return check_launch("mixed_sk_kernel");
}

template <typename T>
int launch_mixed_t(const AttnArgs& ad, const SkArgs& k, const AttnArgs& ap, hipStream_t stream) {
  const bool halves = ad.bs_shift >= 4;
  if (ad.group == 16)
    return halves ? launch_mixed_v<T, 1, true>(ad, k, ap, stream)
                  : launch_mixed_v<T, 1, false>(ad, k, ap, stream);
  return halves ? launch_mixed_v<T, 2, true>(ad, k, ap, stream)
                : launch_mixed_v<T, 2, false>(ad, k, ap, stream);
}

template <typename T, int D, int NT, int PF, bool HALVES, int NW>
int launch_v(const AttnArgs& a, SkArgs k, hipStream_t stream) {
  constexpr int kBlock = 64 * NW;
  k.n_wg = sk_workgroups(D, 16 * NT);
  // a sequence's fixed cost in chunk units of one workgroup's streaming
  // time (at D = 64 twice as many wavefronts would stream a chunk in half
  // the time; at D = 128 the measured optimum of the shape)
  k.seg_cost = D == 128 ? kSkSegCost128(NW) : kSkSegCost * NW / 4;
  if (a.kv8)
    hipLaunchKernelGGL((decode_sk_kernel<T, D, NT, PF, HALVES, true, NW>), dim3(k.n_wg),
                       dim3(kBlock), 0, stream, a, k);
  else
    hipLaunchKernelGGL((decode_sk_kernel<T, D, NT, PF, HALVES, false, NW>), dim3(k.n_wg),
                       dim3(kBlock), 0, stream, a, k);
  return check_launch("decode_sk_kernel");
}

template <typename T, bool HALVES>
int launch_t(const AttnArgs& a, const SkArgs& k, hipStream_t stream) {
  const int nt = a.group / 16;
  // <T, D, NT, PF, HALVES, NW>: one chunk in flight per wavefront (at
  // D = 128 the register budget allows no more; at D = 64 it measured faster
  // than two: cfg4 forced onto this kernel 15.5 against 16.1 us). At D = 128 a
  // batch of decode sequences alone runs 4-wavefront workgroups, one per CU
  // (cfg5: 32.9 against 34.7 us for 8 wavefronts); the decode part of a
  // mixed batch (qfilter 1) 8-wavefront ones, as in the one-launch mixed
  // kernel.
  const bool mixed = a.qfilter == 1;
  if (a.d == 64 && nt == 1) return launch_v<T, 64, 1, 1, HALVES, 4>(a, k, stream);
  if (a.d == 64 && nt == 2) return launch_v<T, 64, 2, 1, HALVES, 4>(a, k, stream);
  if (a.d == 128 && nt == 1)
    return mixed ? launch_v<T, 128, 1, 1, HALVES, 8>(a, k, stream)
                 : launch_v<T, 128, 1, 1, HALVES, 4>(a, k, stream);
  if (a.d == 128 && nt == 2)
    return mixed ? launch_v<T, 128, 2, 1, HALVES, 8>(a, k, stream)
                 : launch_v<T, 128, 2, 1, HALVES, 4>(a, k, stream);
  return fail(PKV_ERR_UNSUPPORTED, "decode_sk: d=%d group=%d", a.d, a.group);
}

}  // namespace

int sk_workgroups(int d, int group) {
  (void)group;
  // one workgroup per CU at D = 128 (4 or 8 wavefronts), two at D = 64
  const int n = (d == 128 ? 1 : 2) * device_cu_count();
  return n < kSkMaxWg ? n : kSkMaxWg;
}

bool mixed_sk_supported(const AttnArgs& ap, int dtype) {
  return (dtype == PKV_DTYPE_BF16 || dtype == PKV_DTYPE_F16) && ap.d == 128 &&
         (ap.group == 16 || ap.group == 32) && !ap.kv8 && ap.k_new && ap.v_new && ap.new_pos &&
         ap.qloc && ap.max_blk >= 1 && ap.num_blocks < (int64_t(1) << 31) &&
         ap.n_seq <= kPrefillFuseMaxSeq && !pool_needs_off64(ap);
}

int launch_mixed_sk(const AttnArgs& ad, const SkArgs& k, const AttnArgs& ap, int dtype,
                    hipStream_t stream) {
  if (!mixed_sk_supported(ap, dtype) || !ad.k_new || !ad.new_pos)
    return fail(PKV_ERR_UNSUPPORTED, "mixed_sk: d=%d group=%d dtype %d", ap.d, ap.group, dtype);
  if (dtype == PKV_DTYPE_BF16) return launch_mixed_t<bf16>(ad, k, ap, stream);
  return launch_mixed_t<f16>(ad, k, ap, stream);
}

int launch_decode_sk(const AttnArgs& a, const SkArgs& k, int dtype, hipStream_t stream) {
  if (a.num_blocks >= (int64_t(1) << 31))
    return fail(PKV_ERR_UNSUPPORTED, "decode_sk: %lld blocks", (long long)a.num_blocks);
  // blocks of 16 tokens or more: per-half chunk addressing (every chunk
  // starts 16-aligned: partitions, shares and table windows are multiples
  // of 32 tokens or of the block size)
  const bool halves = a.bs_shift >= 4;
  if (dtype == PKV_DTYPE_BF16)
    return halves ? launch_t<bf16, true>(a, k, stream) : launch_t<bf16, false>(a, k, stream);
  if (dtype == PKV_DTYPE_F16)
    return halves ? launch_t<f16, true>(a, k, stream) : launch_t<f16, false>(a, k, stream);
  return fail(PKV_ERR_UNSUPPORTED, "decode_sk: dtype %d", dtype);
}

}  // namespace pkv
