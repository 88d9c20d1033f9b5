// Paged MQA attention for query runs longer than one token (prefill and
// chunked prefill) on MFMA: bf16/fp16 storage (or fp8 pools widened in
// LDS), fp32 accumulation, 16 or 32 query heads per KV head, head dim 64 or
// 128. Semantics are those of pagedattn.forward
// (kernels/pagedattn/pagedattn.cu:142-447): query row i of a sequence with
// q_len query tokens and kv_len keys sees keys j < kv_len with, when causal,
// j <= kv_len - q_len + i (bottom-right alignment, :196-207, :315-329); no
// visible key gives a zero row and lse = +inf (:418-446).
//
// Work split. A sequence's query tokens are cut into tiles of TQ tokens (a
// tile = TQ x G rows of one KV head: 8 tokens x 16 heads or 4 x 32; each
// wavefront owns one token's 16-head row tile). Under a causal mask tile t
// sees about (t + 1) TQ keys, so a workgroup takes a PAIR of tiles, t and
// n - 1 - t: every pair of a sequence then walks about the same number of
// key chunks, and the kernel's length is set by the average tile rather
// than the last one. Both tiles of a pair read the same keys (tile t's are a
// prefix of tile n - 1 - t's), so each 32-key chunk is staged in LDS once
// (double-buffered, the next chunks' loads in flight in registers while the
// current one is computed) and used by both tiles' wavefronts: per
// wavefront and chunk, S^T = K Q^T, online softmax with its token's causal
// limit, O^T += V^T P^T (the decode kernels' MFMA steps), once for its
// token of each tile that sees the chunk. Chunks wholly below a token's
// limit skip the score mask.
//
// Grid: one workgroup per pair, 1-D over the pairs of all sequences in
// order (a block-wide scan of the per-sequence pair counts over
// query_start_loc finds a workgroup's sequence and pair); workgroups past
// the last pair, and sequences another launch owns (qfilter), exit. The
// grid is sized by an upper bound, ceil(T / 2 TQ) + n_seq.
//
// This header holds the device code: prefill_pair_body() runs one pair
// workgroup out of the LDS arrays PrefillLds points to, so that the
// stand-alone kernel (prefill_mfma.hip) and the mixed-batch kernel
// (decode_sk.hip), whose workgroups run either a decode share or a prefill
// pair, share it.
#pragma once
#include "mfma_decode_common.h"

#include <type_traits>

namespace pkv {
namespace {

using namespace mfma;

constexpr int kPW = 8;             // wavefronts per workgroup
constexpr int kPBlock = 64 * kPW;  // threads
static_assert(kPBlock == kPrefillFuseMaxSeq, "the fused append's scan is one block");

// Workgroup count bound of a prefill launch over n_tokens query tokens and
// n_seq sequences: ceil(T / 2 TQ) + n_seq pairs (TQ = 8 tokens at 16 query
// heads per kv head, 4 at 32).
inline int64_t prefill_slots(int n_tokens, int n_seq, int group) {
  const int tq = group == 32 ? kPW / 2 : kPW;
  return ((int64_t)n_tokens + 2 * tq - 1) / (2 * tq) + n_seq;
}

// LDS of one pair workgroup: pointers to arrays the kernel declares as
// separate __shared__ objects (after inlining the compiler then knows that
// accesses to different arrays never overlap).
template <int D>
struct PrefillLds {
  static constexpr int kBufBytes = 2 * 2 * ChunkGeo<D>::BYTES;  // [stage][K | V], 16-aligned
  char* buf;
  int* tbl;      // kTblCap entries
  int* scan_sh;  // kPW
  int* sv;       // 4: the pair's sequence, pair index, first query token, query count
  int* dl_seq;   // kPBlock each: fused append, this pair's decode rows
  int* dl_tok;
};

// Pairs of TQ-token tiles of a run of q_len query tokens.
__device__ __forceinline__ int tile_pairs(int q_len, int tq) {
  return ((q_len + tq - 1) / tq + 1) / 2;
}

// A wavefront's two tokens (tile t's and tile n-1-t's), each one 16-head
// row tile: Q^T fragments and online-softmax state as row tiles 0 (token A)
// and 1 (token B), causal key limits (0: no token) and first output rows
// (-1: no token).
template <typename T, int D>
struct PairRows {
  typename Ops<T>::v8 qf[2][D / 32];
  WaveState<2, D / 16> st;
  int lim[2];
  int64_t qrow[2];
};

// Chunk c of the window [lo, hi): BOTH, for both tokens at once (one read
// of each K and V^T fragment for the two; the chunk lies below A's limit),
// else for token B when it sees the chunk.
template <typename T, int D, bool BOTH>
__device__ __forceinline__ void pair_chunk(PairRows<T, D>& x, int c, int lo, int hi,
                                           const ChunkCtx& cx) {
  const int sb = min(x.lim[1], hi);
  if constexpr (BOTH) {
    floatx4 sacc[2][2];
    const int sh[2] = {min(x.lim[0], hi), sb};
    chunk_scores_sub<T, D, 2, 0, 2>(cx, x.qf, sacc);
    chunk_update_sub<T, D, 2, 0, 2, true>(c, cx, sh, sacc, x.st);
  } else {
    if (lo + c * kChunk >= sb) return;  // uniform across the wavefront
    floatx4 sacc[1][2];
    const int sh[1] = {sb};
    chunk_scores_sub<T, D, 2, 1, 1>(cx, x.qf, sacc);
    chunk_update_sub<T, D, 2, 1, 1, true>(c, cx, sh, sacc, x.st);
  }
}

// Row tile k's 16 output rows (and lse) of a wavefront.
template <typename T, int D>
__device__ __forceinline__ void pair_store(PairRows<T, D>& x, int k, const AttnArgs& a,
                                           int lane) {
  constexpr int DT = D / 16;
  x.st.l[k] = head_lanes_sum(x.st.l[k]);
  if (x.qrow[k] < 0) return;  // no token (an active one with no visible key writes zeros)
  const int64_t row = x.qrow[k] + (lane & 15);
  const float L = x.st.l[k];
  const float inv = L > 0.f ? 1.f / L : 0.f;
  T* __restrict__ out = static_cast<T*>(a.out) + row * D + 4 * (lane >> 4);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int e = 0; e < 4; ++e) out[16 * dt + e] = (T)(x.st.o[k][dt][e] * inv);
  if ((lane >> 4) == 0 && a.lse) a.lse[row] = L > 0.f ? (x.st.m[k] + log2f(L)) * kLn2f : INFINITY;
}

// One piece of the fused append: 16 bytes of the K or V row (kv head kvh)
// of token tok, at position pos of sequence s, written with the checks of
// the stand-alone table append (pagedkv append_from_table): a position past
// the table raises SHORT_TABLE, an entry outside [1, blocks) raises
// BAD_BLOCK, and neither writes. phys < 0: read the entry from the table.
template <int D>
__device__ __forceinline__ void append_store(const AttnArgs& a, int s, int pos, int64_t phys,
                                             int kvh, int pc, u32x4 v) {
  constexpr int PPR = D * 2 / 16;  // pieces per K (or V) row
  const int page = pos >> a.bs_shift;
  const bool flag = a.status && pc == 0 && kvh == 0;
  if (pos < 0 || page >= a.max_blk) {
    if (flag) atomicOr(a.status, PKV_STATUS_SHORT_TABLE);
    return;
  }
  if (phys < 0) phys = a.block_tables[(int64_t)s * a.max_blk + page];
  if (phys <= 0 || phys >= a.num_blocks) {
    if (flag) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
    return;
  }
  const bool is_v = pc >= PPR;
  const int64_t slot = (phys << a.bs_shift) + (pos & ((1 << a.bs_shift) - 1));
  char* pool = static_cast<char*>(const_cast<void*>(is_v ? a.v_pool : a.k_pool));
  *reinterpret_cast<u32x4*>(pool + (slot * a.hkv + kvh) * D * 2 + (pc % PPR) * 16) = v;
}

template <int D>
__device__ __forceinline__ u32x4 new_piece(const AttnArgs& a, int tok, int kvh, int pc) {
  constexpr int PPR = D * 2 / 16;
  const char* src = static_cast<const char*>(pc >= PPR ? a.v_new : a.k_new);
  return *reinterpret_cast<const u32x4*>(src + ((int64_t)tok * a.hkv + kvh) * D * 2 +
                                         (pc % PPR) * 16);
}

// Pair `slot` of kv head `kvh` (a workgroup of kPBlock threads).
template <typename T, int D, int WPT, bool OFF64, bool KV8>
__device__ __forceinline__ void prefill_pair_body(AttnArgs a, int slot, int kvh,
                                                  const PrefillLds<D>& sm) {
  using Geo = ChunkGeo<D>;
  constexpr int CPR = Geo::CPR;
  constexpr int PIECES = kChunk * CPR;       // 16-byte pieces of one chunk of K
  constexpr int PER = 2 * PIECES / kPBlock;  // pieces (K and V) per thread
  static_assert(PER >= 1 && 2 * PIECES == PER * kPBlock, "chunk must split evenly");
  constexpr int G = 16 * WPT;
  constexpr int TQ = kPW / WPT;
  char* const buf = sm.buf;
  int* const tbl = sm.tbl;
  int* const scan_sh = sm.scan_sh;
  int& s_seq = sm.sv[0];
  int& s_pair = sm.sv[1];
  int& s_qb = sm.sv[2];
  int& s_ql = sm.sv[3];
  int* const dl_seq = sm.dl_seq;
  int* const dl_tok = sm.dl_tok;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- this workgroup's pair: the slot-th pair of all sequences' pairs.
  // With the fused append (at most kPBlock sequences: one scan block) the
  // scan also numbers the one-token sequences this launch does not attend
  // (a mixed batch's decode rows): pair workgroup p of P appends decode rows
  // [p ND / P, (p + 1) ND / P), and every pair workgroup its own tokens' rows.
  if (a.n_seq <= 0) return;
  const bool fused = a.k_new != nullptr;
  constexpr int PPR = D * 2 / 16;  // 16-byte pieces per K (or V) row
  if (tid == 0) s_seq = -1;  // published by the scan's first barrier
  int run = 0, run_d = 0;
  int my_dex = -1, my_sq = 0, my_tok = 0;  // fused: this thread's decode row
  for (int base = 0; base < a.n_seq; base += kPBlock) {
    const int sq = base + tid;
    int qb = 0, ql = 0;
    if (sq < a.n_seq) {
      qb = a.qloc[sq];
      ql = a.qloc[sq + 1] - qb;
    }
    const bool skip = ql <= 0 || (a.qfilter == 2 && ql == 1);
    // malformed query_start_loc: never index q / out outside [0, T)
    const bool bad = !skip && (qb < 0 || qb + ql > a.n_tokens);
    if (bad && a.status && slot == 0 && kvh == 0) atomicOr(a.status, PKV_STATUS_BAD_QLOC);
    const int np = skip || bad ? 0 : tile_pairs(ql, TQ);
    int ex;
    const int tot = block_scan<kPW>(np, scan_sh, ex);
    if (fused) {
      const int nd = ql == 1 && skip && qb >= 0 && qb < a.n_tokens ? 1 : 0;
      int exd;
      const int totd = block_scan<kPW>(nd, scan_sh, exd);
      if (nd) {
        my_dex = run_d + exd;
        my_sq = sq;
        my_tok = qb;
      }
      run_d += totd;
    }
    if (np > 0 && run + ex <= slot && slot < run + ex + np) {
      s_seq = sq;
      s_pair = slot - run - ex;
      s_qb = qb;
      s_ql = ql;
    }
    run += tot;
    __syncthreads();
    if (!fused && (s_seq >= 0 || run > slot)) break;
  }
  const int s = __builtin_amdgcn_readfirstlane(s_seq);
  if (s < 0) {  // past the last pair
    // fused, and no sequence of the batch has a pair (a max_q_len bound
    // above every query run): pair slot 0 appends the decode rows, each
    // thread its own sequence's (one scan block: a thread holds at most one)
    if (fused && run == 0 && slot == 0 && my_dex >= 0)
      for (int pc = 0; pc < 2 * PPR; ++pc)
        append_store<D>(a, my_sq, a.new_pos[my_sq], -1, kvh, pc, new_piece<D>(a, my_tok, kvh, pc));
    return;
  }
  // fused: this pair's decode rows, listed in LDS (published by the first
  // table window's barrier)
  const int P = run;
  const int dj0 = (int)((int64_t)slot * run_d / P);
  const int nd_rows = (int)((int64_t)(slot + 1) * run_d / P) - dj0;
  if (fused && my_dex >= dj0 && my_dex < dj0 + nd_rows) {
    dl_seq[my_dex - dj0] = my_sq;
    dl_tok[my_dex - dj0] = my_tok;
  }
  const int pair = __builtin_amdgcn_readfirstlane(s_pair);
  const int q_begin = __builtin_amdgcn_readfirstlane(s_qb);
  const int q_len = __builtin_amdgcn_readfirstlane(s_ql);
  const int ntiles = (q_len + TQ - 1) / TQ;
  const int tA = pair;
  const int tB = ntiles - 1 - pair;  // >= tA; == tA: one tile (the middle one)

  // ---- issued together: kv_len, the first table window (entries past
  // the sequence's blocks stay unread: max_blk >= 1 here), both tokens' Q
  int kv_len = ld_meta(a.seq_lens, s);
  // fused: positions [sp, sp + q_len) are this sequence's new rows, read
  // from k_new / v_new (row q_begin + pos - sp) instead of the pool
  const int sp = fused ? ld_meta(a.new_pos, s) : 0;
  // fused: the rows of this pair's own tokens (tile A's, then tile B's),
  // one piece per thread, requested now and written once the first table
  // window is in LDS
  const int nA = min(TQ, q_len - tA * TQ);
  const int n_own = nA + (tB != tA ? min(TQ, q_len - tB * TQ) : 0);
  const int own_u = tid / (2 * PPR);
  const int own_i = own_u < nA ? tA * TQ + own_u : tB * TQ + (own_u - nA);
  const bool own = fused && own_u < n_own;
  u32x4 own_v{};
  if (own) own_v = new_piece<D>(a, q_begin + own_i, kvh, tid % (2 * PPR));
  // fused: this thread's piece of the pair's first kPBlock decode-row
  // pieces, requested once the list is in LDS (the rest at the end)
  const bool dec = fused && tid < nd_rows * 2 * PPR;
  int d_sq = 0, d_pos = -1;
  int64_t d_phys = -1;
  u32x4 d_v{};
  const int32_t* __restrict__ table = a.block_tables + (int64_t)s * a.max_blk;
  const int spec_n = min(a.max_blk, kTblCap);
  const int tspec = table[min(tid, spec_n - 1)];
  const int ti = w / WPT;
  const int h0 = (w % WPT) * 16;
  // a single (middle) tile is token B's, so that B is always the token that
  // sees the most keys
  const int iA = tA * TQ + ti;
  const int iB = tB * TQ + ti;
  const bool actA = tB != tA && iA < q_len;
  const bool actB = iB < q_len;
  const T* __restrict__ q = static_cast<const T*>(a.q);
  PairRows<T, D> X;
  X.qrow[0] = actA ? ((int64_t)(q_begin + iA) * a.hq + kvh * G + h0) : -1;
  X.qrow[1] = actB ? ((int64_t)(q_begin + iB) * a.hq + kvh * G + h0) : -1;
  {
    typename Ops<T>::v8 qa[1][D / 32], qb[1][D / 32];
    load_q<T, D, 1>(qa, q, (int64_t)(q_begin + min(iA, q_len - 1)) * a.hq + kvh * G + h0,
                    lane >> 4, lane & 15);
    load_q<T, D, 1>(qb, q, (int64_t)(q_begin + min(iB, q_len - 1)) * a.hq + kvh * G + h0,
                    lane >> 4, lane & 15);
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      X.qf[0][ks] = qa[0][ks];
      X.qf[1][ks] = qb[0][ks];
    }
  }
  X.st.reset();

  const int cap = a.max_blk << a.bs_shift;
  kv_len = kv_len < cap ? kv_len : cap;
  kv_len = kv_len > 0 ? kv_len : 0;
  const int ctx = a.causal ? max(kv_len - q_len, 0) : 0;
  X.lim[0] = !actA ? 0 : a.causal ? min(kv_len, ctx + iA + 1) : kv_len;
  X.lim[1] = !actB ? 0 : a.causal ? min(kv_len, ctx + iB + 1) : kv_len;
  // the pair's last token's limit bounds every key either tile reads
  const int kv_hi = a.causal ? min(kv_len, ctx + min(q_len, (tB + 1) * TQ)) : kv_len;

  const char* kbase = static_cast<const char*>(a.k_pool);
  const char* vbase = static_cast<const char*>(a.v_pool);
  const int64_t row_stride = (int64_t)a.hkv * D * (KV8 ? 1 : 2);
  const int64_t head_off = (int64_t)kvh * D * (KV8 ? 1 : 2);
  typedef typename PoolPiece<KV8>::type Piece;
  constexpr int PB = PoolPiece<KV8>::kBytes;
  const int bs_mask = (1 << a.bs_shift) - 1;
  ChunkCtx cx;
  cx.tbl = tbl;
  cx.grp = lane >> 4;
  cx.l16 = lane & 15;
  cx.scale_log2 = a.scale_log2;
  bool bad_block = false;

  // this thread's pieces of a chunk: index p of [K pieces | V pieces]
  int prow[PER], pcol[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int p = (tid + k * kPBlock) % PIECES;
    prow[k] = p / CPR;
    pcol[k] = p % CPR;
  }
  auto is_v = [](int k) { return (threadIdx.x + k * kPBlock) >= PIECES; };

  // kTblCap - 1 blocks of tokens per window: a window that starts inside a
  // block still touches at most kTblCap table entries
  const int win = (kTblCap - 1) << a.bs_shift;
  for (int lo = 0; lo < kv_hi; lo += win) {
    const int hi = min(lo + win, kv_hi);
    const int blk_lo = lo >> a.bs_shift;
    const int nblk = ((hi - 1) >> a.bs_shift) + 1 - blk_lo;
    __syncthreads();  // the previous window's table and chunk buffers are no longer read
    if (lo == 0) {
      if (tid < nblk) tbl[tid] = tspec;  // nblk <= spec_n: kv_hi <= max_blk blocks
    } else {
      for (int e = tid; e < nblk; e += kPBlock) tbl[e] = table[blk_lo + e];
    }
    __syncthreads();
    if (lo == 0 && own) {
      const int pos = sp + own_i;
      const int page = pos >> a.bs_shift;
      append_store<D>(a, s, pos, page >= 0 && page < nblk ? tbl[page] : -1, kvh,
                      tid % (2 * PPR), own_v);
    }
    if (lo == 0 && dec) {  // the decode list is published: request row and position
      d_sq = dl_seq[tid / (2 * PPR)];
      d_pos = a.new_pos[d_sq];
      d_v = new_piece<D>(a, dl_tok[tid / (2 * PPR)], kvh, tid % (2 * PPR));
    }
    const int nch = (hi - lo + kChunk - 1) / kChunk;
    // chunk c's pieces into registers; rows past hi re-read the window's
    // last row (masked), rows whose table entry is outside the pool read
    // block 0 and are zeroed when staged. Two register sets alternate, so
    // two chunks are in flight while one is computed; issued for every
    // c < nch + 2 (past the end they re-read chunk nch - 1) so no load sits
    // under a branch.
    Piece rgA[PER], rgB[PER];
    unsigned okA = 0, okB = 0;
    auto issue = [&](int c, Piece (&rg)[PER], unsigned& okm) {
      c = min(c, nch - 1);
      okm = 0;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        int pos = lo + c * kChunk + prow[k];
        pos = pos < hi ? pos : hi - 1;
        const int phys = tbl[(pos >> a.bs_shift) - blk_lo];
        const bool ok = (unsigned)phys < (unsigned)a.num_blocks;
        okm |= (unsigned)ok << k;
        const int slotv = ((ok ? phys : 0) << a.bs_shift) + (pos & bs_mask);
        const char* base = is_v(k) ? vbase : kbase;
        const char* src;
        if constexpr (OFF64)
          src = base + (int64_t)slotv * row_stride + head_off + pcol[k] * PB;
        else
          src = base + ((unsigned)slotv * (unsigned)row_stride + (unsigned)head_off +
                        (unsigned)(pcol[k] * PB));
        if (!KV8 && fused && pos >= sp && pos < sp + q_len) {
          const char* nb = static_cast<const char*>(is_v(k) ? a.v_new : a.k_new);
          src = nb + ((int64_t)(q_begin + pos - sp) * a.hkv + kvh) * D * 2 + pcol[k] * PB;
        }
        rg[k] = *reinterpret_cast<const Piece*>(src);
      }
    };
    // stage chunk c into LDS buffer c & 1 (free: every wavefront passed the
    // previous barrier after computing chunk c - 2), request chunk c + 2
    // into the same registers, then compute chunk c for both tokens
    // chunks [0, cA) are seen by both tokens (A's keys are a prefix of B's),
    // [cA, nch) by B alone: two phases, each with one compute form
    const int sa = min(X.lim[0], hi);
    const int cA = sa > lo ? (sa - lo + kChunk - 1) / kChunk : 0;
    auto step = [&](int c, Piece (&rg)[PER], unsigned& okm, auto both) {
      char* kl = buf + (c & 1) * (2 * Geo::BYTES);
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const bool ok = (okm >> k) & 1;
        bad_block |= !ok;
        u32x4 piece;
        if constexpr (KV8)
          piece = widen8<T>(rg[k]);
        else
          piece = rg[k];
        *reinterpret_cast<u32x4*>(kl + (is_v(k) ? Geo::BYTES : 0) + Geo::off(prow[k], pcol[k])) =
            ok ? piece : u32x4{0u, 0u, 0u, 0u};
      }
      issue(c + 2, rg, okm);
      __syncthreads();  // chunk c is staged; nobody reads the other buffer any more
      cx.kl = kl;
      cx.vl = kl + Geo::BYTES;
      cx.seg_lo = lo;
      pair_chunk<T, D, decltype(both)::value>(X, c, lo, hi, cx);
      if (lo == 0 && c == 0 && dec) {  // its position has arrived: request the table entry
        const int page = d_pos >> a.bs_shift;
        if (d_pos >= 0 && page < a.max_blk)
          d_phys = a.block_tables[(int64_t)d_sq * a.max_blk + page];
      }
    };
    issue(0, rgA, okA);
    issue(1, rgB, okB);
    // chunk c uses register set c & 1 (its loads were issued two chunks
    // earlier into the same set); the branches are uniform
    const std::integral_constant<bool, true> kBoth;
    const std::integral_constant<bool, false> kOne;
    int c = 0;
    for (; c + 1 < cA; c += 2) {
      step(c, rgA, okA, kBoth);
      step(c + 1, rgB, okB, kBoth);
    }
    if (c < cA) {  // odd cA: its last chunk is even, B alone goes on at an odd one
      step(c, rgA, okA, kBoth);
      for (++c; c + 1 < nch; c += 2) {
        step(c, rgB, okB, kOne);
        step(c + 1, rgA, okA, kOne);
      }
      if (c < nch) step(c, rgB, okB, kOne);
    } else {
      for (; c + 1 < nch; c += 2) {
        step(c, rgA, okA, kOne);
        step(c + 1, rgB, okB, kOne);
      }
      if (c < nch) step(c, rgA, okA, kOne);
    }
  }
  if (bad_block && a.status) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);

  // ---- finalise the wavefront's 16 rows of each token
  pair_store<T, D>(X, 0, a, lane);
  pair_store<T, D>(X, 1, a, lane);
  if (fused) {
    if (kv_hi <= 0) {  // no window ran: publish the decode list, request now
      __syncthreads();
      if (dec) {
        d_sq = dl_seq[tid / (2 * PPR)];
        d_pos = a.new_pos[d_sq];
        d_v = new_piece<D>(a, dl_tok[tid / (2 * PPR)], kvh, tid % (2 * PPR));
      }
    }
    if (dec) append_store<D>(a, d_sq, d_pos, d_phys, kvh, tid % (2 * PPR), d_v);
    for (int i = tid + kPBlock; i < nd_rows * 2 * PPR; i += kPBlock) {
      const int r = i / (2 * PPR);
      const int sq = dl_seq[r];
      append_store<D>(a, sq, a.new_pos[sq], -1, kvh, i % (2 * PPR),
                      new_piece<D>(a, dl_tok[r], kvh, i % (2 * PPR)));
    }
  }
}

}  // namespace
}  // namespace pkv
