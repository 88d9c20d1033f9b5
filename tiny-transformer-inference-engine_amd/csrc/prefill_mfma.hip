// Paged MQA attention for query runs longer than one token (prefill and
// chunked prefill) on MFMA: bf16/fp16 storage, fp32 accumulation, 16 or 32
// query heads per KV head, head dim 64 or 128. Semantics are those of
// pagedattn.forward (kernels/pagedattn/pagedattn.cu:142-447): query row i of
// a sequence with q_len query tokens and kv_len keys sees keys
// j < kv_len with, when causal, j <= kv_len - q_len + i (bottom-right
// alignment, :196-207, :315-329); no visible key gives a zero row and
// lse = +inf (:418-446).
//
// A workgroup of 8 wavefronts owns a tile of query tokens of one KV head:
// each token's G heads are covered by WPT wavefronts of NT 16-head row tiles
// each (G = 16 NT WPT; the NT tiles of a wavefront share every K and V^T
// fragment it reads), so a tile holds TQ = 8 / WPT tokens: 8 tokens x 16
// heads, 4 x 32, or 8 x 32 with two row tiles per wavefront, chosen by the
// host for long contexts (fewer K/V re-reads across tiles). The tile's keys are walked
// in 32-token chunks staged once in LDS (double-buffered: the next chunk's
// loads are in flight while the wavefronts compute on the current one) and
// shared by all 8 wavefronts, so each K/V row is read once per tile for
// TQ G rows. Per wavefront and chunk: S^T = K Q^T, online softmax with its
// token's causal limit, O^T += V^T P^T (the decode kernels' MFMA steps).
//
// Grid: one workgroup per tile slot, 1-D. Sequence s owns the slots
// [base_s, base_s + ceil(q_len_s / TQ)), base_s = query_start_loc[s] / TQ + s
// (TQ tokens per tile), a non-decreasing function of s, so
// ceil(T / TQ) + n_seq slots cover every tile and a workgroup finds its
// sequence with one parallel pass over query_start_loc; slots past a
// sequence's tiles, and sequences another launch owns (qfilter), exit.
#include "mfma_decode_common.h"

namespace pkv {
namespace {

using namespace mfma;

constexpr int kPW = 8;             // wavefronts per workgroup
constexpr int kPBlock = 64 * kPW;  // threads

template <typename T, int D, int NT, int WPT, bool OFF64, bool KV8>
__global__ __launch_bounds__(kPBlock, NT == 1 ? 4 : 2) void prefill_mfma_kernel(AttnArgs a) {
  using Geo = ChunkGeo<D>;
  using v8 = typename Ops<T>::v8;
  constexpr int DT = D / 16;
  constexpr int CPR = Geo::CPR;
  constexpr int PIECES = kChunk * CPR;         // 16-byte pieces of one chunk of K
  constexpr int PER = 2 * PIECES / kPBlock;    // pieces (K and V) per thread
  static_assert(PER >= 1 && 2 * PIECES == PER * kPBlock, "chunk must split evenly");
  __shared__ __attribute__((aligned(16))) char buf[2][2 * Geo::BYTES];  // [stage][K | V]
  __shared__ int tbl[kTblCap];
  __shared__ int s_count;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  constexpr int G = 16 * NT * WPT;
  constexpr int TQ = kPW / WPT;
  const int kvh = blockIdx.y;
  const int slot = blockIdx.x;

  // ---- the sequence of this slot: s = #{s : base_s <= slot} - 1
  int cnt = 0;
  for (int s = tid; s < a.n_seq; s += kPBlock) cnt += a.qloc[s] / TQ + s <= slot ? 1 : 0;
  if (tid == 0) s_count = 0;
  __syncthreads();
  if (cnt) atomicAdd(&s_count, cnt);
  __syncthreads();
  const int s = __builtin_amdgcn_readfirstlane(s_count) - 1;
  if (s < 0) return;  // only with a malformed query_start_loc (base_0 = 0 otherwise)
  const int q_begin = ld_meta(a.qloc, s);
  const int q_len = ld_meta(a.qloc, s + 1) - q_begin;
  const int tile = slot - (q_begin / TQ + s);
  if (q_len <= 0 || (a.qfilter == 2 && q_len == 1) || tile * TQ >= q_len) return;
  if (q_begin < 0 || q_begin + q_len > a.n_tokens) {
    // malformed query_start_loc: never index q / out outside [0, T)
    if (a.status && tid == 0) atomicOr(a.status, PKV_STATUS_BAD_QLOC);
    return;
  }
  int kv_len = ld_meta(a.seq_lens, s);
  const int cap = a.max_blk << a.bs_shift;
  kv_len = kv_len < cap ? kv_len : cap;
  kv_len = kv_len > 0 ? kv_len : 0;
  const int ctx = a.causal ? max(kv_len - q_len, 0) : 0;
  const int i0 = tile * TQ;
  const int ntok = min(TQ, q_len - i0);
  // this wavefront's rows: NT 16-head tiles of token i
  const int ti = w / WPT;
  const bool active = ti < ntok;
  const int i = i0 + (active ? ti : 0);
  const int h0 = (w % WPT) * 16 * NT;
  const int lim = !active ? 0 : a.causal ? min(kv_len, ctx + i + 1) : kv_len;
  const int kv_hi = a.causal ? min(kv_len, ctx + i0 + ntok) : kv_len;  // the tile's last token's

  const T* __restrict__ q = static_cast<const T*>(a.q);
  const int64_t qrow0 = (int64_t)(q_begin + i) * a.hq + kvh * G + h0;
  v8 qf[NT][D / 32];
  load_q<T, D, NT>(qf, q, qrow0, lane >> 4, lane & 15);

  const int32_t* __restrict__ table = a.block_tables + (int64_t)s * a.max_blk;
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
  WaveState<NT, DT> st;
  st.reset();
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
    for (int e = tid; e < nblk; e += kPBlock) tbl[e] = table[blk_lo + e];
    __syncthreads();
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
        if constexpr (OFF64) {
          rg[k] = *reinterpret_cast<const Piece*>(base + (int64_t)slotv * row_stride + head_off +
                                                  pcol[k] * PB);
        } else {
          rg[k] = *reinterpret_cast<const Piece*>(
              base + ((unsigned)slotv * (unsigned)row_stride + (unsigned)head_off +
                      (unsigned)(pcol[k] * PB)));
        }
      }
    };
    // stage chunk c into LDS buffer c & 1 (free: every wavefront passed the
    // previous barrier after computing chunk c - 2), request chunk c + 2
    // into the same registers, then compute chunk c
    auto step = [&](int c, Piece (&rg)[PER], unsigned& okm) {
      char* kl = buf[c & 1];
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
      cx.seg_hi = min(lim, hi);
      if (lo + c * kChunk < cx.seg_hi) compute_chunk<T, D, NT>(c, cx, qf, st);
    };
    issue(0, rgA, okA);
    issue(1, rgB, okB);
    for (int c = 0; c < nch; c += 2) {
      step(c, rgA, okA);
      if (c + 1 < nch) step(c + 1, rgB, okB);  // uniform across the workgroup
    }
  }
  if (bad_block && a.status) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);

  // ---- finalise this wavefront's 16 NT rows
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) st.l[nt] = head_lanes_sum(st.l[nt]);
  if (!active) return;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int64_t row = qrow0 + 16 * nt + (lane & 15);
    const float L = st.l[nt];
    const float inv = L > 0.f ? 1.f / L : 0.f;
    T* __restrict__ out = static_cast<T*>(a.out) + row * D + 4 * (lane >> 4);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int e = 0; e < 4; ++e) out[16 * dt + e] = (T)(st.o[nt][dt][e] * inv);
    if ((lane >> 4) == 0 && a.lse)
      a.lse[row] = L > 0.f ? (st.m[nt] + log2f(L)) * kLn2f : INFINITY;
  }
}

template <typename T, int NT, int WPT, bool OFF64>
int launch_nt(const AttnArgs& a, hipStream_t stream) {
  constexpr int tq = kPW / WPT;
  const dim3 grid((a.n_tokens + tq - 1) / tq + a.n_seq, a.hkv);
  if (a.d == 64 && a.kv8)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, 64, NT, WPT, OFF64, true>), grid, dim3(kPBlock),
                       0, stream, a);
  else if (a.d == 64)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, 64, NT, WPT, OFF64, false>), grid, dim3(kPBlock),
                       0, stream, a);
  else if (a.d == 128 && a.kv8)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, 128, NT, WPT, OFF64, true>), grid, dim3(kPBlock),
                       0, stream, a);
  else if (a.d == 128)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, 128, NT, WPT, OFF64, false>), grid,
                       dim3(kPBlock), 0, stream, a);
  else
    return fail(PKV_ERR_UNSUPPORTED, "prefill_mfma: d=%d", a.d);
  return check_launch("prefill_mfma_kernel");
}

template <typename T, bool OFF64>
int launch_t(const AttnArgs& a, hipStream_t stream) {
  if (a.group == 16) return launch_nt<T, 1, 1, OFF64>(a, stream);
  if (a.group == 32 && a.tile_rows == 256) return launch_nt<T, 2, 1, OFF64>(a, stream);
  if (a.group == 32) return launch_nt<T, 1, 2, OFF64>(a, stream);
  return fail(PKV_ERR_UNSUPPORTED, "prefill_mfma: %d query heads per kv head", a.group);
}

}  // namespace

bool prefill_mfma_supported(int dtype, int group, int d) {
  return (dtype == PKV_DTYPE_BF16 || dtype == PKV_DTYPE_F16) && (group == 16 || group == 32) &&
         (d == 64 || d == 128);
}

int launch_prefill_mfma(const AttnArgs& a, int dtype, hipStream_t stream) {
  if (!a.qloc) return fail(PKV_ERR_INVALID, "prefill_mfma: query_start_loc required");
  const int tq = a.group == 32 && a.tile_rows != 256 ? kPW / 2 : kPW;
  const int64_t slots = ((int64_t)a.n_tokens + tq - 1) / tq + a.n_seq;
  if (slots > 0x7fffffff)
    return fail(PKV_ERR_UNSUPPORTED, "prefill_mfma: %lld tile slots", (long long)slots);
  const bool off64 = pool_needs_off64(a);
  if (dtype == PKV_DTYPE_BF16)
    return off64 ? launch_t<bf16, true>(a, stream) : launch_t<bf16, false>(a, stream);
  if (dtype == PKV_DTYPE_F16)
    return off64 ? launch_t<f16, true>(a, stream) : launch_t<f16, false>(a, stream);
  return fail(PKV_ERR_UNSUPPORTED, "prefill_mfma: dtype %d", dtype);
}

}  // namespace pkv
