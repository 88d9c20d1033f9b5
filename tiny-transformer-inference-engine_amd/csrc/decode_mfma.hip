// Paged MQA decode on the gfx950 matrix cores.
//
// One query token per sequence, G = hq / hkv query heads sharing one kv head
// (G = 16 or 32), head dim D = 64 or 128, bf16 or fp16 storage with fp32
// accumulation. Same semantics as the generic kernel (attention.hip) and
// pagedattn.forward (kernels/pagedattn/pagedattn.cu:142-447) for q_len = 1.
//
// Work decomposition: a workgroup of 4 wavefronts owns one (sequence, kv
// head, context partition). Each wavefront walks its own 32-token chunks of
// the partition (chunks w, w+4, ...), so no workgroup barrier sits in the
// main loop. Per chunk a wavefront
//   1. stores the chunk's K and V rows (prefetched into registers during the
//      previous chunk, 16-byte coalesced global loads through the block
//      table) into its private LDS slice, rows padded so that the fragment
//      reads below are bank-conflict free;
//   2. issues the global loads of its next chunk;
//   3. computes S^T = K Q^T with v_mfma_f32_16x16x32 (A = 16 tokens x 32 dims
//      read from LDS, B = Q^T held in registers for the whole partition), so
//      every K row is read once for all G heads;
//   4. updates the online softmax per head in base 2 (each lane owns one
//      head and 8 of the 32 tokens; the row max is a 4-lane xor shuffle);
//   5. computes O^T += V^T P^T with the same instruction: the S^T accumulator
//      layout already is the P^T operand layout (lane = head, 8 tokens), and
//      V^T fragments are gathered from LDS with 16-bit reads.
// At the end the 4 wavefronts merge their (max, sum, O) through LDS, and the
// workgroup writes either the final row (one partition) or a split-K partial
// that merge_kernel (attention.hip) combines.
//
// MFMA operand layouts relied upon (16x16x32, wave64): lane l supplies row
// l%16 of A and column l%16 of B, each with the 8 k-values of group l/16 (the
// k order inside a group is the same for A and B, which is all a reduction
// needs); lane l receives D[4*(l/16) + r][l%16] for r = 0..3.
#include "pkv_internal.h"

namespace pkv {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct MfmaOps;
template <>
struct MfmaOps<bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ floatx4 mma(v8 a, v8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct MfmaOps<f16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ floatx4 mma(v8 a, v8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

constexpr int kWaves = 4;
constexpr int kBlock = 64 * kWaves;
constexpr int kTblCap = 256;  // block-table entries of one partition kept in LDS
constexpr float kLn2f = 0.6931471805599453f;

// LDS geometry of one 32-token chunk of K (or V) rows, D bf16/fp16 each.
// Rows are padded by 16 bytes (PITCH = 2D + 16): row r starts 4r (mod 64)
// banks further on for D = 128 (36r for D = 64), so the 16 rows an MFMA
// fragment read touches at one 16-byte piece land on distinct bank groups,
// and so do the 4 row groups of a V^T gather. Every fragment address is then
// one base register plus an immediate offset.
template <int D>
struct ChunkGeo {
  static constexpr int CPR = D / 8;                 // 16-byte pieces per row
  static constexpr int ROW_BYTES = D * 2;
  static constexpr int PITCH = ROW_BYTES + 16;
  static constexpr int ROWS_PER_LOAD = 64 / CPR;    // rows one wave load covers
  static constexpr int NPL = kChunk / ROWS_PER_LOAD;  // loads per lane per tensor
  static constexpr int BYTES = kChunk * PITCH;
  static_assert(ROWS_PER_LOAD >= 1 && 64 % CPR == 0, "D must be 64 or 128");
  static __device__ __forceinline__ int off(int r, int c) { return r * PITCH + (c << 4); }
};

// K and V rows of one 32-token chunk held in registers between its loads
// and its LDS stores; bit j of `valid` clears row load j (bad table entry).
template <int NPL>
struct ChunkRegs {
  u32x4 k[NPL];
  u32x4 v[NPL];
  unsigned valid;
};

// Per-wavefront view of the pool used by the loader.
struct PoolView {
  const char* kbase;
  const char* vbase;
  int64_t row_stride;  // bytes per pool slot (hkv * d * 2)
  int64_t head_off;    // byte offset of this kv head inside a slot
  int num_blocks;
  int bs_shift;
};

// Branch-free loads of one chunk starting at token `cb`: rows past `seg_hi`
// re-read the segment's last row (their scores are masked to -inf later, so
// they contribute exactly 0); rows whose table entry is outside the pool read
// block 0 and are zeroed when staged. Nothing here consumes a load result,
// so the loads stay in flight until the chunk is staged PF chunks later.
// OFF64 = false when every byte offset of the pool fits in 31 bits: the
// load is then a uniform 64-bit base plus a 32-bit per-lane offset.
template <class Geo, int NPL, bool OFF64>
__device__ __forceinline__ void load_chunk(ChunkRegs<NPL>& r, const PoolView& pv,
                                           const int* tbl, int blk_lo, int cb,
                                           int seg_hi, int prow, int pcol) {
  const int bs_mask = (1 << pv.bs_shift) - 1;
  unsigned vmask = 0;
#pragma unroll
  for (int j = 0; j < NPL; ++j) {
    int pos = cb + prow + j * Geo::ROWS_PER_LOAD;
    pos = pos < seg_hi ? pos : seg_hi - 1;
    const int phys = tbl[(pos >> pv.bs_shift) - blk_lo];
    const bool ok = (unsigned)phys < (unsigned)pv.num_blocks;
    vmask |= (unsigned)ok << j;
    const int slot = ((ok ? phys : 0) << pv.bs_shift) + (pos & bs_mask);
    if constexpr (OFF64) {
      const int64_t off = (int64_t)slot * pv.row_stride + pv.head_off + pcol * 16;
      r.k[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pv.kbase + off));
      r.v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pv.vbase + off));
    } else {
      const unsigned off = (unsigned)slot * (unsigned)pv.row_stride +
                           (unsigned)pv.head_off + (unsigned)(pcol * 16);
      r.k[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pv.kbase + off));
      r.v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(pv.vbase + off));
    }
  }
  r.valid = vmask;
}

// PF = chunks each wavefront keeps in flight in registers; OCC = wavefronts
// per SIMD the register budget is sized for (2 x PF x 16 KiB of loads per
// CU in flight either way for the D = 128 / 32-head variant).
// QLDS: Q^T fragments are re-read from LDS per chunk instead of being held
// in registers (for the variant whose registers are otherwise exhausted).
template <typename T, int D, int NT, int PF, int OCC, bool OFF64, bool QLDS>
__global__ __launch_bounds__(kBlock, OCC) void decode_mfma_kernel(AttnArgs a) {
  using Ops = MfmaOps<T>;
  using v8 = typename Ops::v8;
  using Geo = ChunkGeo<D>;
  constexpr int G = 16 * NT;     // heads of the group
  constexpr int KS = D / 32;     // k-steps of QK
  constexpr int DT = D / 16;     // 16-wide column tiles of PV
  constexpr int NPL = Geo::NPL;
  constexpr int WAVE_BYTES = 2 * Geo::BYTES;
  constexpr int OPITCH = D + 4;  // floats; +4 spreads head rows over banks
  constexpr int MERGE_BYTES = kWaves * G * OPITCH * 4;
  constexpr int Q_OFF = kWaves * WAVE_BYTES;           // Q^T rows, laid out like K
  constexpr int MAIN_BYTES = Q_OFF + (QLDS ? G * D * 2 : 0);
  constexpr int LDS_BYTES = MAIN_BYTES > MERGE_BYTES ? MAIN_BYTES : MERGE_BYTES;
  static_assert(!QLDS || G == kChunk, "Q staging reuses the 32-row chunk geometry");
  static_assert(MERGE_BYTES <= LDS_BYTES, "merge staging must fit the K/V region");
  __shared__ __attribute__((aligned(16))) char lds[LDS_BYTES];
  __shared__ float ml_lds[kWaves][G][2];
  __shared__ int tbl[kTblCap];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int grp = lane >> 4;   // k-group of this lane in MFMA operands
  const int l16 = lane & 15;
  // sequence fastest: consecutive workgroups go to different XCDs, so the
  // partitions of short and long sequences spread over all of them
  const int part = blockIdx.y;
  const int s = blockIdx.x / a.hkv;
  const int kvh = blockIdx.x - s * a.hkv;
  TileGeom g;
  if (!tile_geom(a, s, 0, G, g)) return;
  if (part >= g.nparts) return;
  const int kv_lo = part * g.part_len;
  const int kv_hi = min(kv_lo + g.part_len, g.kv_limit);
  const int bs_shift = a.bs_shift;

  const int32_t* __restrict__ table = a.block_tables + (int64_t)s * a.max_blk;

  // Q^T fragments for the whole partition: head 16*nt + l16, dims of piece
  // 4*ks + grp
  const T* __restrict__ q = static_cast<const T*>(a.q);
  const int64_t qrow0 = (int64_t)g.q_begin * a.hq + kvh * G;
  v8 qf[QLDS ? 1 : NT][QLDS ? 1 : KS];
  char* ql = lds + Q_OFF;
  if constexpr (QLDS) {
    // G rows of D elements, laid out like a K chunk
    for (int i = threadIdx.x; i < G * Geo::CPR; i += kBlock) {
      const int row = i / Geo::CPR, pc = i % Geo::CPR;
      *reinterpret_cast<u32x4*>(ql + Geo::off(row, pc)) =
          *reinterpret_cast<const u32x4*>(q + (qrow0 + row) * D + pc * 8);
    }
  } else {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        qf[nt][ks] = *reinterpret_cast<const v8*>(q + (qrow0 + 16 * nt + l16) * D +
                                                 (4 * ks + grp) * 8);
  }
  auto qfrag = [&](int nt, int ks) -> v8 {
    if constexpr (QLDS)
      return *reinterpret_cast<const v8*>(ql + Geo::off(16 * nt + l16, 4 * ks + grp));
    else
      return qf[nt][ks];
  };

  PoolView pv;
  pv.kbase = static_cast<const char*>(a.k_pool);
  pv.vbase = static_cast<const char*>(a.v_pool);
  pv.row_stride = (int64_t)a.hkv * D * 2;
  pv.head_off = (int64_t)kvh * D * 2;
  pv.num_blocks = (int)a.num_blocks;
  pv.bs_shift = bs_shift;
  char* kl = lds + w * WAVE_BYTES;
  char* vl = kl + Geo::BYTES;
  const int prow = lane / Geo::CPR;   // first row this lane loads
  const int pcol = lane % Geo::CPR;   // its 16-byte piece within the row
  bool bad_block = false;

  floatx4 o[NT][DT];
  float m[NT], l[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m[nt] = -INFINITY;
    l[nt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[nt][dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  ChunkRegs<NPL> rb[PF];
  int seg_lo = kv_lo, seg_hi = kv_lo, blk_lo = 0, nchunks = 0;

  // one chunk: registers -> LDS slice, refill the registers with the chunk
  // PF steps ahead, then QK / softmax / PV out of LDS
  auto process = [&](ChunkRegs<NPL>& r, int c, bool refill) {
    asm volatile("" ::: "memory");
    const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
      const int row = prow + j * Geo::ROWS_PER_LOAD;
      const bool ok = (r.valid >> j) & 1;
      bad_block |= !ok;
      *reinterpret_cast<u32x4*>(kl + Geo::off(row, pcol)) = ok ? r.k[j] : zero;
      *reinterpret_cast<u32x4*>(vl + Geo::off(row, pcol)) = ok ? r.v[j] : zero;
    }
    if (refill)
      load_chunk<Geo, NPL, OFF64>(r, pv, tbl, blk_lo, seg_lo + (c + kWaves * PF) * kChunk, seg_hi,
                           prow, pcol);
    // the slice is private to this wavefront: waiting for its own LDS
    // writes is the only synchronisation the reads below need
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");

    // S^T = K Q^T, tokens 16h + 4*grp + r of this chunk for head 16nt + l16
    floatx4 sacc[NT][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v8 kf[KS];
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kf[ks] = *reinterpret_cast<const v8*>(kl + Geo::off(16 * h + l16, 4 * ks + grp));
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        floatx4 acc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) acc = Ops::mma(kf[ks], qfrag(nt, ks), acc);
        sacc[nt][h] = acc;
      }
    }

    // online softmax (base 2); P^T operand = this lane's 8 probabilities
    const int cb = seg_lo + c * kChunk;
    v8 pf[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float sv[8];
      float mx = -INFINITY;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int pos = cb + 16 * h + 4 * grp + rr;
          const float x = pos < seg_hi ? sacc[nt][h][rr] * a.scale_log2 : -INFINITY;
          sv[4 * h + rr] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m[nt], mx);
      const float ref = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m[nt] - ref);
      float ps = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = exp2f(sv[e] - ref);
        ps += p;
        pf[nt][e] = (T)p;
      }
      l[nt] = l[nt] * alpha + ps;
      m[nt] = m_new;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) o[nt][dt] *= alpha;
    }

    // O^T += V^T P^T; V^T fragment: dims 16dt + l16, the same 8 tokens
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      v8 vf;
      const int d = 16 * dt + l16;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int tok = (e < 4 ? 0 : 16) + 4 * grp + (e & 3);
        vf[e] = *reinterpret_cast<const T*>(vl + Geo::off(tok, d >> 3) + (d & 7) * 2);
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) o[nt][dt] = Ops::mma(vf, pf[nt], o[nt][dt]);
    }
  };

  // The partition is walked in segments of at most kTblCap table entries
  // (one segment unless a sequence outgrew the planned bound); each
  // segment's table slice is staged in LDS by one coalesced read.
  const int seg_len = kTblCap << bs_shift;
  for (seg_lo = kv_lo; seg_lo < kv_hi; seg_lo += seg_len) {
    seg_hi = min(seg_lo + seg_len, kv_hi);
    blk_lo = seg_lo >> bs_shift;
    const int nblk = ((seg_hi - 1) >> bs_shift) + 1 - blk_lo;
    __syncthreads();  // previous segment's table no longer read
    for (int i = threadIdx.x; i < nblk; i += kBlock) tbl[i] = table[blk_lo + i];
    __syncthreads();
    nchunks = (seg_hi - seg_lo + kChunk - 1) / kChunk;
#pragma unroll
    for (int b = 0; b < PF; ++b)
      if (w + kWaves * b < nchunks)
        load_chunk<Geo, NPL, OFF64>(rb[b], pv, tbl, blk_lo, seg_lo + (w + kWaves * b) * kChunk,
                             seg_hi, prow, pcol);
    int c = w;
    // steady state: every buffer holds a loaded chunk and is refilled with
    // the chunk PF steps ahead. No branch depends on the data, so the
    // compiler's wait counts stay exact: staging buffer b waits only for
    // buffer b's loads while the other buffers' loads stay in flight.
    for (; c + kWaves * (2 * PF - 1) < nchunks; c += kWaves * PF) {
#pragma unroll
      for (int b = 0; b < PF; ++b) process(rb[b], c + kWaves * b, true);
    }
    // drain: at most 2*PF - 1 chunks left for this wavefront
#pragma unroll
    for (int b = 0; b < PF; ++b)
      if (c + kWaves * b < nchunks)
        process(rb[b], c + kWaves * b, c + kWaves * (b + PF) < nchunks);
    c += kWaves * PF;
#pragma unroll
    for (int b = 0; b < PF; ++b)
      if (c + kWaves * b < nchunks) process(rb[b], c + kWaves * b, false);
  }
  if (bad_block && a.status) atomicOr(a.status, PKV_STATUS_BAD_BLOCK);

  // ---- merge the 4 wavefronts' partial states through LDS ----
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    l[nt] += __shfl_xor(l[nt], 16);
    l[nt] += __shfl_xor(l[nt], 32);
  }
  __syncthreads();  // every wavefront is done with its K/V slice
  float* ob = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<floatx4*>(ob + (w * G + 16 * nt + l16) * OPITCH + 16 * dt + 4 * grp) =
          o[nt][dt];
  if (grp == 0) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      ml_lds[w][16 * nt + l16][0] = m[nt];
      ml_lds[w][16 * nt + l16][1] = l[nt];
    }
  }
  __syncthreads();

  T* __restrict__ out = static_cast<T*>(a.out);
  const int64_t unit = (int64_t)blockIdx.x * a.parts_max + part;
  for (int idx = threadIdx.x; idx < G * D / 4; idx += kBlock) {
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
    const int64_t qrow = qrow0 + head;
    if (g.nparts == 1) {
      const float inv = L > 0.f ? 1.f / L : 0.f;
      T* dst = out + qrow * D + d0;
      dst[0] = (T)(acc[0] * inv);
      dst[1] = (T)(acc[1] * inv);
      dst[2] = (T)(acc[2] * inv);
      dst[3] = (T)(acc[3] * inv);
      if (d0 == 0 && a.lse) a.lse[qrow] = L > 0.f ? (M + log2f(L)) * kLn2f : INFINITY;
    } else {
      *reinterpret_cast<floatx4*>(a.ws_o + (unit * G + head) * D + d0) = acc;
      if (d0 == 0) {
        a.ws_ml[(unit * G + head) * 2 + 0] = M;
        a.ws_ml[(unit * G + head) * 2 + 1] = L;
      }
    }
  }
}

template <typename T, bool OFF64>
int launch_t(const AttnArgs& a, const AttnPlan& p, hipStream_t stream) {
  const dim3 grid(a.n_seq * a.hkv, p.parts_max);
  const int nt = a.group / 16;
  // <T, D, NT, PF, OCC, OFF64>: every variant runs two wavefronts per SIMD;
  // the D = 128, 32-head one has room for one chunk in flight per wavefront,
  // the others for two
  if (a.d == 64 && nt == 1)
    hipLaunchKernelGGL((decode_mfma_kernel<T, 64, 1, 2, 2, OFF64, false>), grid, dim3(kBlock), 0, stream, a);
  else if (a.d == 64 && nt == 2)
    hipLaunchKernelGGL((decode_mfma_kernel<T, 64, 2, 2, 2, OFF64, false>), grid, dim3(kBlock), 0, stream, a);
  else if (a.d == 128 && nt == 1)
    hipLaunchKernelGGL((decode_mfma_kernel<T, 128, 1, 1, 2, OFF64, false>), grid, dim3(kBlock), 0, stream, a);
  else if (a.d == 128 && nt == 2)
    hipLaunchKernelGGL((decode_mfma_kernel<T, 128, 2, 1, 2, OFF64, false>), grid, dim3(kBlock), 0, stream, a);
  else
    return fail(PKV_ERR_UNSUPPORTED, "decode_mfma: d=%d group=%d", a.d, a.group);
  return check_launch("decode_mfma_kernel");
}

}  // namespace

bool decode_mfma_supported(int dtype, int max_q_len, int group, int d) {
  return (dtype == PKV_DTYPE_BF16 || dtype == PKV_DTYPE_F16) && max_q_len == 1 &&
         (group == 16 || group == 32) && (d == 64 || d == 128);
}

int launch_decode_mfma(const AttnArgs& a, const AttnPlan& p, int dtype,
                       hipStream_t stream) {
  if (a.num_blocks >= (int64_t(1) << 31))
    return fail(PKV_ERR_UNSUPPORTED, "decode_mfma: %lld blocks", (long long)a.num_blocks);
  const int64_t pool_bytes = a.num_blocks * ((int64_t)a.hkv * a.d * 2) << a.bs_shift;
  const bool off64 = pool_bytes >= (int64_t(1) << 31);
  if (dtype == PKV_DTYPE_BF16)
    return off64 ? launch_t<bf16, true>(a, p, stream) : launch_t<bf16, false>(a, p, stream);
  if (dtype == PKV_DTYPE_F16)
    return off64 ? launch_t<f16, true>(a, p, stream) : launch_t<f16, false>(a, p, stream);
  return fail(PKV_ERR_UNSUPPORTED, "decode_mfma: dtype %d", dtype);
}

}  // namespace pkv
