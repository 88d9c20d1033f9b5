// Paged MQA decode on the gfx950 matrix cores, one workgroup per context
// partition (the split-K form; decode_sk.hip is the persistent form).
//
// One query token per sequence, G = hq / hkv query heads sharing one kv head
// (G = 16 or 32), head dim D = 64 or 128, bf16 or fp16 storage with fp32
// accumulation. Same semantics as the generic kernel (attention.hip) and
// pagedattn.forward (kernels/pagedattn/pagedattn.cu:142-447) for q_len = 1.
//
// A workgroup of 4 wavefronts owns one (sequence, kv head, partition); each
// wavefront walks its own 32-token chunks of the partition (chunks w, w+4,
// ...) through the pipeline of mfma_decode_common.h, so no workgroup barrier
// sits in the main loop. At the end the 4 wavefronts merge their
// (max, sum, O) through LDS and the workgroup writes the final row (one
// partition) or a split-K partial. With arrival counters (AttnArgs::merge_ctr)
// the partition that completes a sequence's count merges its partials in
// the same launch; without them (prefill tiles, very large batches)
// merge_kernel (attention.hip) combines them in a second launch.
// The grid is sequence-fastest: workgroups are dispatched round-robin over
// the XCDs, so consecutive workgroups of different sequences spread the
// partitions of short and long sequences over all of them.
#include "mfma_decode_common.h"

namespace pkv {
namespace {

using namespace mfma;

constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;
static_assert(kBlock >= kTblCap, "one thread per table entry of a window");

// PF = chunks each wavefront keeps in flight in registers; OCC = wavefronts
// per SIMD the register budget is sized for; APP = the fused append of
// a.k_new / a.v_new at a.new_pos (compiled out of the plain attention); KV8 =
// fp8 pools (rows widened to T when staged in LDS).
template <typename T, int D, int NT, int PF, int OCC, bool HALVES, bool APP, bool KV8>
__global__ __launch_bounds__(kBlock, OCC) void decode_mfma_kernel(AttnArgs a) {
  using Geo = ChunkGeo<D>;
  using v8 = typename Ops<T>::v8;
  constexpr int G = 16 * NT;     // heads of the group
  constexpr int DT = D / 16;     // 16-wide column tiles of PV
  constexpr int WAVE_BYTES = 2 * Geo::BYTES;
  constexpr int OPITCH = D + 4;  // floats; +4 spreads head rows over banks
  constexpr int MERGE_BYTES = kWaves * G * OPITCH * 4;
  constexpr int MAIN_BYTES = kWaves * WAVE_BYTES;
  constexpr int LDS_BYTES = MAIN_BYTES > MERGE_BYTES ? MAIN_BYTES : MERGE_BYTES;
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
  __shared__ float ml_lds[kWaves][G][2];
  __shared__ int tbl[kTblCap];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (scalar)
  const int grp = lane >> 4;
  const int l16 = lane & 15;
  const int part = blockIdx.y;
  const int s = blockIdx.x / a.hkv;
  const int kvh = blockIdx.x - s * a.hkv;
  const int32_t* __restrict__ table = a.block_tables + (int64_t)s * a.max_blk;
  const T* __restrict__ q = static_cast<const T*>(a.q);
  // Requested before the sequence's metadata arrives: the partition's first
  // table window at the planned partition length (one entry per thread,
  // entries past the table's end clamped and unused) and the Q rows of query
  // token s (a decode batch's query_start_loc is 0, 1, 2, ...; when it is
  // not, the rows are requested again once it has arrived).
  const int spec_blk0 = (part * a.part_tokens) >> a.bs_shift;
  const int tspec = table[max(0, min(spec_blk0 + (int)threadIdx.x, a.max_blk - 1))];
  v8 qf[NT][D / 32];
  if (s < a.n_tokens) load_q<T, D, NT>(qf, q, (int64_t)s * a.hq + kvh * G, grp, l16);
  // fused append: the new row's position and its pieces are requested with
  // Q (the pieces of query token s, again once query_start_loc has arrived
  // if it is not s), so the append adds no round trip ahead of the chunks
  int new_pos_s = -1;
  u32x4 new_piece{};
  if constexpr (APP) {
    new_pos_s = a.new_pos[s];
    if (s < a.n_tokens) new_piece = load_new_row<D>(a, s, kvh, threadIdx.x);
  }
  TileGeom g;
  if (!tile_geom(a, s, 0, G, g)) return;
  if (part >= g.nparts) return;
  const int kv_lo = part * g.part_len;
  const int kv_hi = min(kv_lo + g.part_len, g.kv_limit);
  const int64_t qrow0 = (int64_t)g.q_begin * a.hq + kvh * G;
  if (g.q_begin != s) {  // uniform
    load_q<T, D, NT>(qf, q, qrow0, grp, l16);
    if constexpr (APP) new_piece = load_new_row<D>(a, g.q_begin, kvh, threadIdx.x);
  }
  // the speculative window is this partition's first one unless the
  // sequence outgrew the planned bound (longer partitions)
  const bool spec_ok = g.part_len == a.part_tokens;

  PoolView pv;
  pv.kbase = static_cast<const char*>(a.k_pool);
  pv.vbase = static_cast<const char*>(a.v_pool);
  pv.row_stride = (int64_t)a.hkv * D * (KV8 ? 1 : 2);
  pv.head_off = (int64_t)kvh * D * (KV8 ? 1 : 2);
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
  WaveState<NT, DT> st;
  st.reset();
  // fused append: the partition holding the new row's position stages it
  // from k_new / v_new; the last partition writes it into the pool
  __shared__ __attribute__((aligned(16))) char new_lds[2 * Geo::ROW_BYTES];
  NewRow nr;
  nr.pos = -1;
  nr.lds = new_lds;
  int new_pos = -1;
  bool new_write = false, new_pending = false;  // pending: row buffer still to fill
  if constexpr (APP) {
    new_pos = new_pos_s;
    const bool new_here = new_pos >= kv_lo && new_pos < kv_hi;
    new_write = part == g.nparts - 1;
    if (new_here) nr.pos = new_pos;
    new_pending = new_here || new_write;
  }
  int last_blk_lo = 0, last_nblk = 0;

  // walk the partition in windows of kTblCap - 1 blocks of tokens, so that a
  // window starting inside a block still touches at most kTblCap table
  // entries (one window unless a sequence outgrew the planned bound)
  const int win = (kTblCap - 1) << a.bs_shift;
  for (int lo = kv_lo; lo < kv_hi; lo += win) {
    cx.seg_lo = lo;
    cx.seg_hi = min(lo + win, kv_hi);
    cx.blk_lo = lo >> a.bs_shift;
    const int nblk = ((cx.seg_hi - 1) >> a.bs_shift) + 1 - cx.blk_lo;
    __syncthreads();  // previous window's table no longer read
    const bool spec = spec_ok && lo == kv_lo;
    if (APP && new_pending) {
      const u32x4 piece = new_piece;
      if (spec) {
        if ((int)threadIdx.x < nblk) tbl[threadIdx.x] = tspec;
      } else {
        for (int i = threadIdx.x; i < nblk; i += kBlock) tbl[i] = table[cx.blk_lo + i];
      }
      put_new_row<D>(new_lds, piece, threadIdx.x);
      new_pending = false;
    } else if (spec) {
      if ((int)threadIdx.x < nblk) tbl[threadIdx.x] = tspec;
    } else {
      for (int i = threadIdx.x; i < nblk; i += kBlock) tbl[i] = table[cx.blk_lo + i];
    }
    __syncthreads();
    run_chunks<T, D, NT, PF, HALVES, APP, KV8>(w, kWaves, cx, pv, qf, st, bad_block, nr);
    last_blk_lo = cx.blk_lo;
    last_nblk = nblk;
  }
  if (bad_block && a.status) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);
  if (APP && new_write) {
    if (new_pending) put_new_row<D>(new_lds, new_piece, threadIdx.x);
    // each thread stores the piece it put into the buffer itself
    store_new_row<T, D, KV8>(new_lds, a, s, kvh, new_pos, tbl, last_blk_lo, last_nblk,
                             threadIdx.x);
  }

  // ---- merge the 4 wavefronts' partial states through LDS ----
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    st.l[nt] = head_lanes_sum(st.l[nt]);
  }
  __syncthreads();  // every wavefront is done with its K/V slice
  float* ob = reinterpret_cast<float*>(lds);
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

  T* __restrict__ out = static_cast<T*>(a.out);
  const int64_t unit = (int64_t)blockIdx.x * a.parts_max + part;
  using Combine = WaveCombine<G, D, kWaves, kBlock>;
  {
    Combine cb;
    cb.run(ob, ml_lds, threadIdx.x);
    const int64_t qrow = qrow0 + cb.head;
    if (g.nparts == 1) {
#pragma unroll
      for (int q = 0; q < Combine::NQ; ++q) {
        T* dst = out + qrow * D + cb.col(q);
        dst[0] = (T)(cb.acc[q][0] * cb.inv);
        dst[1] = (T)(cb.acc[q][1] * cb.inv);
        dst[2] = (T)(cb.acc[q][2] * cb.inv);
        dst[3] = (T)(cb.acc[q][3] * cb.inv);
      }
      if (cb.cq == 0 && a.lse) a.lse[qrow] = cb.L > 0.f ? (cb.M + log2f(cb.L)) * kLn2f : INFINITY;
    } else {
      const int64_t prow = unit * G + cb.head;
      if (a.merge_ctr) {
        // O / sum rounded to T (a weighted mean of value rows, so within
        // their range; bf16 keeps fp32's exponent range) and the fp32
        // (max, sum): half the partial traffic of unnormalised fp32 rows.
        // Written through to memory: the merging workgroup may sit on
        // another XCD.
        uint16_t* po16 = reinterpret_cast<uint16_t*>(a.ws_o) + prow * D;
#pragma unroll
        for (int q = 0; q < Combine::NQ; ++q) st_agent64(po16 + cb.col(q), pack4<T>(cb.acc[q], cb.inv));
        if (cb.cq == 0) {
          const float2 ml = make_float2(cb.M, cb.L);
          uint64_t bm;
          __builtin_memcpy(&bm, &ml, 8);
          st_agent64(a.ws_ml + prow * 2, bm);
        }
      } else {
#pragma unroll
        for (int q = 0; q < Combine::NQ; ++q)
          *reinterpret_cast<floatx4*>(a.ws_o + prow * D + cb.col(q)) = cb.acc[q];
        if (cb.cq == 0) {
          a.ws_ml[prow * 2 + 0] = cb.M;
          a.ws_ml[prow * 2 + 1] = cb.L;
        }
      }
    }
  }
  if (!a.merge_ctr || g.nparts == 1) return;

  // ---- in-kernel split-K merge: once its partial stores have completed,
  // each partition counts itself in; the one that brings the count to
  // nparts merges every partition (each thread one head and the columns of
  // the wavefront combination above; loads issued in batches of 8
  // partitions before any is consumed), writes the rows and resets the
  // counter for the next call. No workgroup waits for another.
  __shared__ int s_last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    int* ctr = a.merge_ctr + blockIdx.x;
    const int old = fetch_add_agent(ctr, 1);
    s_last = old == g.nparts - 1;
    if (s_last) __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // a counter that started at c != 0 shows a value outside [0, nparts) to
    // at least one partition (the largest it sees is c + nparts - 1, the
    // smallest c): never silent
    if ((old < 0 || old >= g.nparts) && a.status) atomicOr(a.status, PKV_STATUS_DIRTY_WORKSPACE);
  }
  __syncthreads();
  if (!s_last) return;
  const int64_t unit0 = (int64_t)blockIdx.x * a.parts_max;
  constexpr int kMB = 8;
  constexpr int NQ = Combine::NQ;
  const int head = threadIdx.x / Combine::TPH;
  const int cq = threadIdx.x - head * Combine::TPH;
  float M = -INFINITY, L = 0.f;
  floatx4 acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = floatx4{0.f, 0.f, 0.f, 0.f};
  const uint16_t* po16 = reinterpret_cast<const uint16_t*>(a.ws_o);
  for (int p0 = 0; p0 < g.nparts; p0 += kMB) {
    float2 ml[kMB];
    uint64_t oo[kMB][NQ];
#pragma unroll
    for (int j = 0; j < kMB; ++j) {
      const int64_t row = (unit0 + min(p0 + j, g.nparts - 1)) * G + head;
      ml[j] = *reinterpret_cast<const float2*>(a.ws_ml + row * 2);
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        oo[j][q] = *reinterpret_cast<const uint64_t*>(po16 + row * D + 4 * (cq + Combine::TPH * q));
    }
#pragma unroll
    for (int j = 0; j < kMB; ++j) {
      if (p0 + j >= g.nparts || ml[j].x == -INFINITY) continue;
      const float Mn = fmaxf(M, ml[j].x);
      const float sa = exp2f(M - Mn);
      const float wl = ml[j].y * exp2f(ml[j].x - Mn);  // this partial's weight
      L = L * sa + wl;
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        acc[q] = acc[q] * sa + unpack4<T>(oo[j][q]) * wl;
      M = Mn;
    }
  }
  const int64_t qrow = qrow0 + head;
  const float inv = L > 0.f ? 1.f / L : 0.f;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    T* dst = out + qrow * D + 4 * (cq + Combine::TPH * q);
    dst[0] = (T)(acc[q][0] * inv);
    dst[1] = (T)(acc[q][1] * inv);
    dst[2] = (T)(acc[q][2] * inv);
    dst[3] = (T)(acc[q][3] * inv);
  }
  if (cq == 0 && a.lse) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2f : INFINITY;
}

// <T, D, NT, PF, OCC, HALVES, APP, KV8>: the register budget of two
// wavefronts per SIMD at D = 128, four at D = 64 (the kernel needs about
// 100 VGPRs there; the tighter target measured the 12-layer config-4 step
// 156.4 against 157.6 us)
template <typename T, int D, int NT, int PF, bool HALVES, bool KV8>
void launch_k(const AttnArgs& a, dim3 grid, hipStream_t stream) {
  constexpr int kOcc = D == 64 ? 4 : 2;
  if (a.new_pos)
    hipLaunchKernelGGL((decode_mfma_kernel<T, D, NT, PF, kOcc, HALVES, true, KV8>), grid,
                       dim3(kBlock), 0, stream, a);
  else
    hipLaunchKernelGGL((decode_mfma_kernel<T, D, NT, PF, kOcc, HALVES, false, KV8>), grid,
                       dim3(kBlock), 0, stream, a);
}
template <typename T, int D, int NT, int PF, bool HALVES>
void launch_v(const AttnArgs& a, dim3 grid, hipStream_t stream) {
  if (a.kv8)
    launch_k<T, D, NT, PF, HALVES, true>(a, grid, stream);
  else
    launch_k<T, D, NT, PF, HALVES, false>(a, grid, stream);
}

template <typename T, bool HALVES>
int launch_t(const AttnArgs& a, const AttnPlan& p, hipStream_t stream) {
  const dim3 grid(a.n_seq * a.hkv, p.parts_max);
  const int nt = a.group / 16;
  // one chunk in flight per wavefront: at D = 128 the register budget
  // allows no more; at D = 64 it measured fastest (cfg4: 12.8 against 13.4
  // us for two and 14.1 / 14.2 us for three / four; the whole grid is
  // resident at once, and fewer registers leave room for more wavefronts
  // per SIMD)
  if (a.d == 64 && nt == 1)
    launch_v<T, 64, 1, 1, HALVES>(a, grid, stream);
  else if (a.d == 64 && nt == 2)
    launch_v<T, 64, 2, 1, HALVES>(a, grid, stream);
  else if (a.d == 128 && nt == 1)
    launch_v<T, 128, 1, 1, HALVES>(a, grid, stream);
  else if (a.d == 128 && nt == 2)
    launch_v<T, 128, 2, 1, HALVES>(a, grid, stream);
  else
    return fail(PKV_ERR_UNSUPPORTED, "decode_mfma: d=%d group=%d", a.d, a.group);
  return check_launch("decode_mfma_kernel");
}

}  // namespace

bool decode_mfma_supported(int dtype, int max_q_len, int group, int d) {
  return (dtype == PKV_DTYPE_BF16 || dtype == PKV_DTYPE_F16) && max_q_len == 1 &&
         (group == 16 || group == 32) && (d == 64 || d == 128);
}

bool pool_needs_off64(const AttnArgs& a) {
  const int64_t pool_bytes = (a.num_blocks * ((int64_t)a.hkv * a.d * (a.kv8 ? 1 : 2)))
                            << a.bs_shift;
  return pool_bytes >= (int64_t(1) << 31);
}

int launch_decode_mfma(const AttnArgs& a, const AttnPlan& p, int dtype,
                       hipStream_t stream) {
  if (a.num_blocks >= (int64_t(1) << 31))
    return fail(PKV_ERR_UNSUPPORTED, "decode_mfma: %lld blocks", (long long)a.num_blocks);
  // blocks of 16 tokens or more: per-half chunk addressing (every chunk
  // starts 16-aligned: partitions, shares and table windows are multiples
  // of 32 tokens or of the block size)
  const bool halves = a.bs_shift >= 4;
  if (dtype == PKV_DTYPE_BF16)
    return halves ? launch_t<bf16, true>(a, p, stream) : launch_t<bf16, false>(a, p, stream);
  if (dtype == PKV_DTYPE_F16)
    return halves ? launch_t<f16, true>(a, p, stream) : launch_t<f16, false>(a, p, stream);
  return fail(PKV_ERR_UNSUPPORTED, "decode_mfma: dtype %d", dtype);
}

}  // namespace pkv
